// gguf_mv.hip — matvec over GGUF bytes with fp32 activations: the arithmetic
// of the reference's matvec_q8_0 / matvec_q4_K (src/kernels/matvec.cpp:62-142:
// y[m] += sum over the row of dequantized weight * x, no activation
// quantization), as a weight stream on the vector ALUs.  No MFMA: with one fp32
// activation vector there is no second operand dimension to fill a matrix
// instruction, and every weight needs its own fp32 multiply-add anyway.
//
// Thread layout: a workgroup owns R consecutive rows.  Each thread owns one
// weight-block column of the row (Q8_0: one 32-element block; Q4_K: one
// 64-element quarter of a super-block) and holds that column's activations in
// registers for the workgroup's whole life; P threads share a column and take
// every P-th row of the tile.  Per row a thread produces one partial sum,
// parked in LDS; a wave then adds a row's partials (wave-level DPP sum) and
// accumulates into y.
//
// Q8_0 (34-byte blocks, 2-byte aligned): the tile's bytes are one contiguous
// range (rows are contiguous in GGUF), loaded with 16-byte coalesced loads
// (non-temporal: every byte is used once) and staged in LDS, where each
// thread reads its block at its 2-byte-aligned offset.  Needs K % 256 == 0 so
// that rows start 16-byte aligned.
// Q4_K (144-byte super-blocks, 16-byte aligned): each thread loads its own
// 16-byte header and 32 bytes of nibbles straight from HBM (lanes of a wave
// cover consecutive 32-byte runs); the per-sub-block form
// y = sum (d*sc) * sum(q x) - (dmin*m) * sum(x) uses activation sums computed
// once per thread.
#include <algorithm>
#include <cstdlib>

#include "common.hpp"

namespace ec {

namespace {

typedef uint32_t gu32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt16(const uint8_t* p) {
    const gu32x4 v = __builtin_nontemporal_load((const gu32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Rows' partial sums red[rr][0 .. ncol) -> y[r0 + rr] = y0[rr] + sum, one wave
// per row.  y0 holds the rows' previous y values, read at kernel start (no
// dependent global load at the end of the workgroup: 10.3 -> 9.9 us at
// 9216 x 2560); nothing else writes these rows during the kernel.
__device__ __forceinline__ void reduce_rows(const float* red, const float* y0, uint32_t ncol, uint32_t nr,
                                            float* __restrict__ y, uint32_t r0) {
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    for (uint32_t rr = w; rr < nr; rr += nw) {
        float s = 0.0f;
        for (uint32_t c = lane; c < ncol; c += 64) s += red[rr * ncol + c];
        s = wave_sum(s);
        if (lane == 0) y[r0 + rr] = y0[rr] + s;
    }
}

constexpr int kQ8Stage = 8;  // 16-byte tile chunks per thread (R rows x K/32*34 bytes <= 8 * 16 * threads)

// grid.x = ceil(M / R); blockDim = P * nb (nb = K/32 blocks per row).  The
// tile's bytes and the thread's 32 activations are all in flight before the
// first use.
__global__ __launch_bounds__(1024) void k_gguf_q8_0_f32(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                        float* __restrict__ y, uint32_t M, uint32_t nb, uint32_t P,
                                                        uint32_t R) {
    extern __shared__ uint8_t lds[];
    const uint32_t t = threadIdx.x, T = blockDim.x;
    const uint32_t b = t % nb, ph = t / nb;
    const size_t rowbytes = (size_t)nb * 34;
    const uint32_t r0 = blockIdx.x * R, nr = min(R, M - r0);
    float* red = (float*)(lds + ((R * rowbytes + 15) & ~(size_t)15));
    float* y0 = red + (size_t)R * nb;  // previous y of the tile's rows (R <= blockDim.x)
    const float yp = t < nr ? y[r0 + t] : 0.0f;
    const uint8_t* src = W + (size_t)r0 * rowbytes;
    const uint32_t n16 = (uint32_t)(nr * rowbytes / 16);
    uint4 v[kQ8Stage];
#pragma unroll
    for (int i = 0; i < kQ8Stage; ++i) {
        const uint32_t c = t + i * T;
        v[i] = c < n16 ? ld_nt16(src + 16 * (size_t)c) : make_uint4(0u, 0u, 0u, 0u);
    }
    float xv[32];
    const float4* xb = (const float4*)(x + 32 * b);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = xb[i];
        xv[4 * i] = f.x, xv[4 * i + 1] = f.y, xv[4 * i + 2] = f.z, xv[4 * i + 3] = f.w;
    }
#pragma unroll
    for (int i = 0; i < kQ8Stage; ++i) {
        const uint32_t c = t + i * T;
        if (c < n16) *(uint4*)(lds + 16 * (size_t)c) = v[i];
    }
    __syncthreads();
    for (uint32_t rr = ph; rr < nr; rr += P) {
        const uint16_t* bp = (const uint16_t*)(lds + rr * rowbytes + 34 * (size_t)b);
        const float d = h2f(bp[0]);
        float bs = 0.0f;  // the block's sum in element order, as the reference's inner loop
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint32_t w2 = bp[1 + k];
            bs = fmaf((float)(int8_t)(w2 & 0xFF), xv[2 * k], bs);
            bs = fmaf((float)(int8_t)(w2 >> 8), xv[2 * k + 1], bs);
        }
        red[rr * nb + b] = d * bs;
    }
    if (t < nr) y0[t] = yp;
    __syncthreads();
    reduce_rows(red, y0, nb, nr, y, r0);
}

// grid.x = ceil(M / R), R = RPT * P rows (RPT rows per thread, each one 16-byte
// header + 32 bytes of nibbles loaded straight from HBM); blockDim = P * nq
// (nq = 4 * K/256 quarters per row).
template <int RPT>
__global__ __launch_bounds__(1024) void k_gguf_q4_K_f32(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                        float* __restrict__ y, uint32_t M, uint32_t nsb, uint32_t P,
                                                        uint32_t R) {
    extern __shared__ uint8_t lds[];
    float* red = (float*)lds;
    const uint32_t t = threadIdx.x, nq = 4 * nsb;
    const uint32_t q = t % nq, ph = t / nq, sb = q / 4, g = q % 4;
    const size_t rowbytes = (size_t)nsb * 144;
    const uint32_t r0 = blockIdx.x * R, nr = min(R, M - r0);
    float* y0 = red + (size_t)R * nq;  // previous y of the tile's rows (R <= blockDim.x)
    const float yp = t < nr ? y[r0 + t] : 0.0f;
    uint4 hd[RPT], q0[RPT], q1[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const uint32_t rr = ph + i * P;
        const bool ok = rr < nr;
        const uint8_t* bp = W + (size_t)(r0 + (ok ? rr : 0)) * rowbytes + 144 * (size_t)sb;
        hd[i] = ok ? *(const uint4*)bp : make_uint4(0u, 0u, 0u, 0u);
        q0[i] = ok ? ld_nt16(bp + 16 + 32 * g) : make_uint4(0u, 0u, 0u, 0u);
        q1[i] = ok ? ld_nt16(bp + 32 + 32 * g) : make_uint4(0u, 0u, 0u, 0u);
    }
    // activations of the quarter, in the reference's position order: pair 0 of
    // the 64-group at positions 0-15 (low nibbles of bytes 0-15) and 32-47
    // (their high nibbles), pair 1 at 16-31 and 48-63 (bytes 16-31)
    float xv[64];
    const float4* xb = (const float4*)(x + 256 * sb + 64 * g);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 f = xb[i];
        xv[4 * i] = f.x, xv[4 * i + 1] = f.y, xv[4 * i + 2] = f.z, xv[4 * i + 3] = f.w;
    }
    float xs0 = 0.0f, xs1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        xs0 += xv[j] + xv[32 + j];
        xs1 += xv[16 + j] + xv[48 + j];
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const uint32_t rr = ph + i * P;
        if (rr >= nr) break;
        const uint32_t scw[3] = {hd[i].y, hd[i].z, hd[i].w};  // scales[0..11]
        auto byte = [&](int k) -> uint32_t { return (scw[k >> 2] >> (8 * (k & 3))) & 0xFFu; };
        uint32_t sc0, mn0, sc1, mn1;
        const int s0 = 2 * (int)g, s1 = s0 + 1;
        // 6-bit scale / min unpack (src/kernels/quant.cpp:222-242)
        if (s0 < 4) {
            sc0 = byte(s0) & 63u, mn0 = byte(s0 + 4) & 63u;
            sc1 = byte(s1) & 63u, mn1 = byte(s1 + 4) & 63u;
        } else {
            sc0 = (byte(s0 + 4) & 0x0Fu) | ((byte(s0 - 4) >> 6) << 4);
            mn0 = (byte(s0 + 4) >> 4) | ((byte(s0) >> 6) << 4);
            sc1 = (byte(s1 + 4) & 0x0Fu) | ((byte(s1 - 4) >> 6) << 4);
            mn1 = (byte(s1 + 4) >> 4) | ((byte(s1) >> 6) << 4);
        }
        const float d = h2f(hd[i].x & 0xFFFF), dmin = h2f(hd[i].x >> 16);
        const uint32_t qw[8] = {q0[i].x, q0[i].y, q0[i].z, q0[i].w, q1[i].x, q1[i].y, q1[i].z, q1[i].w};
        float S0 = 0.0f, S1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // bytes 0-15: pair 0
            const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S0 = fmaf((float)((lo >> (8 * e)) & 0xFF), xv[4 * k + e], S0);
                S0 = fmaf((float)((hi >> (8 * e)) & 0xFF), xv[32 + 4 * k + e], S0);
            }
        }
#pragma unroll
        for (int k = 4; k < 8; ++k) {  // bytes 16-31: pair 1
            const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S1 = fmaf((float)((lo >> (8 * e)) & 0xFF), xv[4 * k + e], S1);
                S1 = fmaf((float)((hi >> (8 * e)) & 0xFF), xv[32 + 4 * k + e], S1);
            }
        }
        red[rr * nq + q] = (d * (float)sc0) * S0 - (dmin * (float)mn0) * xs0 + (d * (float)sc1) * S1 -
                           (dmin * (float)mn1) * xs1;
    }
    if (t < nr) y0[t] = yp;
    __syncthreads();
    reduce_rows(red, y0, nq, nr, y, r0);
}

uint32_t gcd32(uint32_t a, uint32_t b) {
    while (b) {
        const uint32_t r = a % b;
        a = b;
        b = r;
    }
    return a;
}

}  // namespace

// Launch the GGUF fp32 kernel for fmt, or return EC_ERR_UNSUPPORTED when the
// shape does not fit it (the caller then uses the per-row kernel; so does
// EC_GGUF_KERNEL=rows, for comparison).
int gguf_mv_fast(int fmt, const uint8_t* W, const float* x, float* y, uint32_t M, uint32_t K, hipStream_t st) {
    static const bool rows = [] {
        const char* v = getenv("EC_GGUF_KERNEL");
        return v && v[0] == 'r';
    }();
    if (rows || ((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return EC_ERR_UNSUPPORTED;
    if (fmt == EC_Q8_0) {
        const uint32_t nb = K / 32;
        if (K % 256 || nb > 1024) return EC_ERR_UNSUPPORTED;
        uint32_t P = 64 / gcd32(nb, 64);  // P * nb a whole number of waves
        while (P > 1 && P * nb > 1024) P /= 2;
        const uint32_t T = P * nb;
        const size_t rowbytes = (size_t)nb * 34;
        // rows per workgroup: a multiple of P whose bytes fit the staging registers and ~48 KB of LDS
        uint32_t R = P;
        while ((R + P) * rowbytes <= (size_t)kQ8Stage * 16 * T && (R + P) * (rowbytes + 4 * nb) <= 48 * 1024) R += P;
        if (R * rowbytes > (size_t)kQ8Stage * 16 * T) return EC_ERR_UNSUPPORTED;
        const size_t lds = ((R * rowbytes + 15) & ~(size_t)15) + (size_t)R * nb * 4 + (size_t)R * 4;
        if (R > T) return EC_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(k_gguf_q8_0_f32, dim3((M + R - 1) / R), dim3(T), lds, st, W, x, y, M, nb, P, R);
        return EC_OK;
    }
    if (fmt == EC_Q4_K) {
        const uint32_t nsb = K / 256, nq = 4 * nsb;
        if (nq > 1024) return EC_ERR_UNSUPPORTED;
        uint32_t P = 64 / gcd32(nq, 64);
        while (P > 1 && P * nq > 1024) P /= 2;
        // two rows per thread (both rows' loads in flight) unless that leaves
        // fewer than 512 workgroups
        const uint32_t rpt = (M + 2 * P - 1) / (2 * P) >= 512 ? 2 : 1;
        const uint32_t R = rpt * P;
        const dim3 grid((M + R - 1) / R), blk(P * nq);
        const size_t lds = (size_t)R * nq * 4 + (size_t)R * 4;
        if (R > P * nq) return EC_ERR_UNSUPPORTED;
        if (rpt == 2) hipLaunchKernelGGL(k_gguf_q4_K_f32<2>, grid, blk, lds, st, W, x, y, M, nsb, P, R);
        else hipLaunchKernelGGL(k_gguf_q4_K_f32<1>, grid, blk, lds, st, W, x, y, M, nsb, P, R);
        return EC_OK;
    }
    return EC_ERR_UNSUPPORTED;
}

}  // namespace ec
