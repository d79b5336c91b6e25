// gguf_mv.hip — matvec over GGUF bytes with fp32 activations: the arithmetic
// of the reference's matvec_q8_0 / matvec_q4_K (src/kernels/matvec.cpp:62-142:
// y[m] += sum over the row of dequantized weight * x, no activation
// quantization), as a weight stream on the vector ALUs.  No MFMA: with one fp32
// activation vector there is no second operand dimension to fill a matrix
// instruction, and every weight needs its own fp32 multiply-add anyway.
//
// Thread layout: a workgroup owns R consecutive rows.  Each thread owns one
// 64-element column of the row (Q8_0: a pair of 32-element blocks; Q4_K: a
// quarter of a super-block) and holds that column's activations in registers
// for the workgroup's whole life; P threads share a column and take every
// P-th row of the tile.  Per row a thread produces one partial sum, parked in
// LDS; then a group of up to 64 threads adds a row's partials with lane
// exchanges and one thread accumulates the row into y.
//
// Q8_0 (34-byte blocks, 2-byte aligned; K % 64 == 0): a block pair is 68
// bytes at a dword-aligned offset, loaded by its thread straight from HBM
// (four 16-byte loads and a dword per row, lanes of a wave covering
// consecutive pairs) with x staged in LDS as for Q4_K; each weight byte is
// converted by its own byte select, so block 0's 2-byte offset costs nothing.
// Q4_K (144-byte super-blocks, 16-byte aligned): each thread loads its own
// 16-byte header and 32 bytes of nibbles straight from HBM for each of its
// RPT rows (lanes of a wave cover consecutive 32-byte runs), all issued
// first; the workgroup stages x once in LDS (quarters 272 bytes apart, so 16
// consecutive lanes' 16-byte reads fall in distinct banks) and each thread
// copies its quarter to registers for its rows -- x is read from L2 once per
// workgroup of R = RPT * P rows instead of once per thread; the
// per-sub-block form y = sum (d*sc) * sum(q x) - (dmin*m) * sum(x) uses
// activation sums computed once per thread.
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

// Hides v's known-zero bits from the optimizer (an empty asm, no
// instruction): with four nibbles masked into the low halves of four bytes,
// (float)((v >> 8n) & 0xFF) then selects the single v_cvt_f32_ubyte<n>
// instead of a 4-bit field extract plus a convert.
__device__ __forceinline__ void hide_bits(uint32_t& v) { asm("" : "+v"(v)); }

// Sum of v over this lane's aligned group of G consecutive lanes (G a power
// of two <= 64, uniform); every lane of the group receives the total.
__device__ __forceinline__ float sum_group(float v, uint32_t G) {
    if (G >= 2) v += lane_xor<1>(v);
    if (G >= 4) v += lane_xor<2>(v);
    if (G >= 8) v += lane_xor<4>(v);
    if (G >= 16) v += lane_xor<8>(v);
    if (G >= 32) v += lane_xor<16>(v);
    if (G >= 64) v += lane_xor<32>(v);
    return v;
}

// Rows' values red[rr][0 .. ncol) -> y[r0 + rr] = yp + sum for rr < nr: the G
// consecutive threads rr*G .. rr*G + G-1 (G a power of two <= 64, G * R <=
// blockDim) add every G-th value, then exchange; thread rr*G stores.  yp is
// the row's previous y, loaded by every thread of the group at kernel start
// (y[r0 + min(t / G, nr - 1)]: no dependent global load at the end of the
// workgroup); nothing else writes these rows during the kernel.  One store
// per row (a wave per row with scattered single-float stores cost 1.8 us of
// 8.2 at Q4_K 9216 x 2560).
__device__ __forceinline__ void row_sums_store(const float* red, uint32_t ncol, uint32_t nr, uint32_t G, float yp,
                                               float* __restrict__ y, uint32_t r0) {
    const uint32_t t = threadIdx.x, rr = t / G, G0 = rr * G;
    float acc = 0.0f;
    if (rr < nr)
        for (uint32_t c = t - G0; c < ncol; c += G) acc += red[rr * ncol + c];
    acc = sum_group(acc, G);
    if (t == G0 && rr < nr) y[r0 + rr] = yp + acc;
}

// Block-pair form (K % 64 == 0): thread column c owns blocks 2c and 2c + 1
// of its rows, 68 bytes at a dword-aligned offset (the row stride nb * 34 is
// a multiple of 4), loaded straight from memory as four 16-byte loads and a
// dword per row, all RPT rows issued before any use.  Element j of block 0
// is byte 2 + j of those 17 dwords and of block 1 byte 36 + j; each is
// converted with its own byte select, so the 2-byte offset of block 0 costs
// nothing.  x is staged in LDS once per workgroup, read into registers by
// each thread for its column, and the rows' pair values are summed by
// row_sums_store.  Issue order as in the Q4_K kernel below: x's loads, the
// previous y, then the weights, all unconditional, so the x staging and
// barrier overlap the weights' latency.  x in LDS as pairs of 64 floats 65
// apart: the compiler re-reads x from LDS inside the row loop (it keeps the
// kernel at ~60 registers), and with an odd stride consecutive lanes (pairs)
// read distinct banks, at compile-time offsets.  (Pairs 68 floats apart, for
// 16-byte reads: lanes 16 apart shared banks, 1.4 M conflict cycles per
// 9216 x 2560 launch.)
constexpr uint32_t kQ8XStride = 65;

size_t q8_f32_lds_bytes(uint32_t nc, uint32_t R) { return ((size_t)nc * kQ8XStride + 4 + (size_t)R * nc + 1) * 4; }

typedef uint32_t gu32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// nc_magic = ceil(2^32 / nc): t / nc == umulhi(t, nc_magic) for t, nc < 2^10.
template <int RPT, int XPT>
__global__ __launch_bounds__(1024) void k_gguf_q8_0_f32_pairs(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, uint32_t M, uint32_t nc,
    uint32_t P, uint32_t R, uint32_t G, uint32_t nc_magic) {
    extern __shared__ uint8_t lds[];
    const uint32_t t = threadIdx.x, T = blockDim.x;
    constexpr uint32_t XS = kQ8XStride;
    float* xs = (float*)lds;  // [nc][XS], then a 4-float spare slot
    float* red = xs + (size_t)nc * XS + 4;  // [R][nc] + 1
    const uint32_t ph0 = __umulhi(t, nc_magic), c = t - ph0 * nc;
    const uint32_t ph = min(ph0, P - 1);  // padding threads: c < nc, ph0 >= P
    const size_t rowbytes = (size_t)nc * 68;
    const uint32_t r0 = blockIdx.x * R, nr = min(R, M - r0), n4 = 16 * nc;
    float4 xf[XPT];  // float4s t, t + T, ... of x
#pragma unroll
    for (int j = 0; j < XPT; ++j) xf[j] = ((const float4*)x)[min(t + j * T, n4 - 1)];
    const float yp = y[r0 + min(t / G, nr - 1)];
    __builtin_amdgcn_sched_barrier(0);  // keep x's loads ahead of the weights'
    uint32_t w[RPT][17];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const uint32_t rr = ph + i * P;
        const uint8_t* bp = W + (size_t)(r0 + (rr < nr ? rr : 0)) * rowbytes + 68 * (size_t)c;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const gu32x4a4 v = *(const gu32x4a4*)(bp + 16 * k);
            w[i][4 * k] = v.x, w[i][4 * k + 1] = v.y, w[i][4 * k + 2] = v.z, w[i][4 * k + 3] = v.w;
        }
        w[i][16] = *(const uint32_t*)(bp + 64);
    }
    // x -> LDS: float4 c4 (elements 4(c4 % 16) .. +3 of pair c4 / 16)
    // (unconditional: float4s past x's end go to the spare slot -- a branch
    // here lets the compiler sink the weights' loads below the barrier)
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const uint32_t c4 = t + j * T;
        float* o = xs + (c4 < n4 ? (c4 / 16) * XS + 4 * (c4 % 16) : nc * XS);
        o[0] = xf[j].x, o[1] = xf[j].y, o[2] = xf[j].z, o[3] = xf[j].w;
    }
    __syncthreads();
    float xv[64];
    const float* xq = xs + c * XS;
#pragma unroll
    for (int i = 0; i < 64; ++i) xv[i] = xq[i];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        // branch-free: a row past the tile's end (rr >= nr) sums row r0's
        // bytes into the spare slot or a slot that is never read
        const uint32_t rr = ph + i * P;
        const float d0 = h2f(w[i][0] & 0xFFFF), d1 = h2f(w[i][8] >> 16);
        // each block's sum in element order, as the reference's inner loop
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            s0 = fmaf((float)(int8_t)(w[i][(2 + j) >> 2] >> (8 * ((2 + j) & 3))), xv[j], s0);
            s1 = fmaf((float)(int8_t)(w[i][9 + (j >> 2)] >> (8 * (j & 3))), xv[32 + j], s1);
        }
        red[ph0 < P ? rr * nc + c : R * nc] = d0 * s0 + d1 * s1;
    }
    __syncthreads();
    row_sums_store(red, nc, nr, G, yp, y, r0);
}

template <int RPT>
int launch_q8_f32_x(uint32_t xpt, dim3 grid, dim3 blk, size_t lds, hipStream_t st, const uint8_t* W, const float* x,
                    float* y, uint32_t M, uint32_t nc, uint32_t P, uint32_t R, uint32_t G, uint32_t mg) {
    switch (xpt) {
#define EC_Q8F(X)                                                                                             \
    case X:                                                                                                   \
        hipLaunchKernelGGL((k_gguf_q8_0_f32_pairs<RPT, X>), grid, blk, lds, st, W, x, y, M, nc, P, R, G, mg); \
        break;
        EC_Q8F(1) EC_Q8F(2) EC_Q8F(4) EC_Q8F(8) EC_Q8F(16)
#undef EC_Q8F
        default: return EC_ERR_UNSUPPORTED;
    }
    return EC_OK;
}

// grid.x = ceil(M / R), R = RPT * P rows; blockDim T = P * nq rounded up to
// whole waves (nq = 4 * K/256 quarters per row, P a power of two).  Thread t
// takes quarter q = t % nq of rows ph + i*P (ph = t / nq, i < RPT): per row a
// 16-byte header and 32 bytes of nibbles loaded straight from HBM, so the
// lanes of one load instruction cover consecutive quarters of one row.
// Threads t >= P * nq only pad the last wave.  The workgroup's 16 * nq float4s
// of x are XPT per thread (T * XPT >= 16 * nq).  LDS (floats): x as nq
// quarters of 68 (64 + 4 padding, where padding threads' stores land), x's
// pair sums [nq][2], then the rows' quarter values [R][nq] and a spare slot.
//
// Issue order matters: vector-memory loads complete in order, so x's loads go
// first and the weights' after them, all unconditional (a row past the
// tile's end re-reads row r0 and is never used) -- the wait before x's LDS
// store then covers x alone, and the staging, barrier and LDS reads overlap
// the weights' HBM latency.
//
// x's pair sums come from the staging registers: 16 consecutive lanes hold
// one quarter's 16 float4s, so two lane-exchange sums give both pairs.  The
// row sums: G = T / R (a power of two, at most 64) consecutive threads share
// a row, each adding every G-th quarter value, then lane exchanges; thread
// rr * G stores y for row rr -- one store per row, after all loads.
constexpr uint32_t kQ4XStride = 68;  // floats per staged quarter (272 bytes)

// Four rows' loads (48 registers) beside the 64 activations need more than
// the 128 registers a 1024-thread workgroup allows: RPT = 4 is bounded at 768
// threads (up to 168 registers, spill-free).
template <int RPT>
constexpr int q4_f32_max_threads() { return RPT == 4 ? 768 : 1024; }

size_t q4_f32_lds_bytes(uint32_t nq, uint32_t R) {
    return ((size_t)nq * (kQ4XStride + 2) + (size_t)R * nq + 1) * 4;
}

// 6-bit scale and min of sub-blocks 2g and 2g + 1 from the 12 scale bytes
// (w0 = bytes 0-3, w1 = 4-7, w2 = 8-11), the packing of src/kernels/quant.cpp:222-242:
// sub-block j < 4: scale = byte j & 63, min = byte j+4 & 63; j >= 4: scale =
// (byte j+4 & 15) | (byte j-4 >> 6) << 4, min = (byte j+4 >> 4) | (byte j >> 6) << 4.
// Both cases read bytes 2(g & 1) + s of w0, w1 (and w2), branch-free.
__device__ __forceinline__ void q4_scale_min(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t g, uint32_t& sc0,
                                             uint32_t& mn0, uint32_t& sc1, uint32_t& mn1) {
    const uint32_t sh = 16 * (g & 1);
    const uint32_t a = w0 >> sh, b = w1 >> sh, c = w2 >> sh;
    const bool hi = g >= 2;
    sc0 = hi ? (c & 15u) | ((a >> 2) & 48u) : a & 63u;
    mn0 = hi ? ((c >> 4) & 15u) | ((b >> 2) & 48u) : b & 63u;
    sc1 = hi ? ((c >> 8) & 15u) | ((a >> 10) & 48u) : (a >> 8) & 63u;
    mn1 = hi ? ((c >> 12) & 15u) | ((b >> 10) & 48u) : (b >> 8) & 63u;
}

// nq_magic = ceil(2^32 / nq): t / nq == umulhi(t, nq_magic) exactly for
// t, nq < 2^10 (the rounding error t * (nq_magic - 2^32/nq) / 2^32 < 2^-22
// is below the 1/nq gap to the next integer).
template <int RPT, int XPT>
__global__ __launch_bounds__(q4_f32_max_threads<RPT>()) void k_gguf_q4_K_f32(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, uint32_t M, uint32_t nsb,
    uint32_t P, uint32_t R, uint32_t G, uint32_t nq_magic) {
    extern __shared__ uint8_t lds[];
    const uint32_t t = threadIdx.x, T = blockDim.x, nq = 4 * nsb;
    float* xs = (float*)lds;
    float2* xsum = (float2*)(xs + (size_t)nq * kQ4XStride);
    float* red = (float*)(xsum + nq);  // [R][nq] + 1
    const uint32_t ph0 = __umulhi(t, nq_magic), q = t - ph0 * nq;
    const uint32_t ph = min(ph0, P - 1), sb = q / 4, g = q % 4;  // padding threads: q < nq, ph0 >= P
    const size_t rowbytes = (size_t)nsb * 144;
    const uint32_t r0 = blockIdx.x * R, nr = min(R, M - r0), n4 = 16 * nq;
    float4 xf[XPT];  // float4s t, t + T, ... of x
#pragma unroll
    for (int j = 0; j < XPT; ++j) xf[j] = ((const float4*)x)[min(t + j * T, n4 - 1)];
    const float yp = y[r0 + min(t / G, nr - 1)];
    __builtin_amdgcn_sched_barrier(0);  // keep x's loads ahead of the weights'
    uint4 hd[RPT], q0[RPT], q1[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const uint32_t rr = ph + i * P;
        const uint8_t* bp = W + (size_t)(r0 + (rr < nr ? rr : 0)) * rowbytes + 144 * (size_t)sb;
        hd[i] = *(const uint4*)bp;
        q0[i] = ld_nt16(bp + 16 + 32 * g);
        q1[i] = ld_nt16(bp + 32 + 32 * g);
    }
    // x -> LDS, quarter c (64 floats) at c * 68 floats, float4s past x's end
    // into the last quarter's padding; float4 k of a quarter (lane % 16 == k)
    // is in pair 0 for k & 4 == 0 (positions 0-15, 32-47), pair 1 otherwise
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const uint32_t c4 = t + j * T;
        const uint32_t o = c4 < n4 ? (c4 / 16) * kQ4XStride + 4 * (c4 % 16) : (nq - 1) * kQ4XStride + 64;
        *(float4*)(xs + o) = xf[j];
        float ps = (xf[j].x + xf[j].y) + (xf[j].z + xf[j].w);
        ps += lane_xor<1>(ps);
        ps += lane_xor<2>(ps);
        ps += lane_xor<8>(ps);
        if (c4 < n4 && (c4 & 11) == 0) ((float*)xsum)[2 * (c4 / 16) + ((c4 >> 2) & 1)] = ps;
    }
    __syncthreads();
    // the thread's quarter, in the reference's position order: pair 0 of the
    // 64-group at positions 0-15 (low nibbles of bytes 0-15) and 32-47 (their
    // high nibbles), pair 1 at 16-31 and 48-63 (bytes 16-31)
    float xv[64];
    const float4* xq = (const float4*)(xs + q * kQ4XStride);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 f = xq[i];
        xv[4 * i] = f.x, xv[4 * i + 1] = f.y, xv[4 * i + 2] = f.z, xv[4 * i + 3] = f.w;
    }
    const float2 xm = xsum[q];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        // branch-free: a row past the tile's end (rr >= nr) sums row r0's
        // bytes, and its value is never read -- a branch here would let the
        // compiler sink the weights' loads below the barrier
        const uint32_t rr = ph + i * P;
        uint32_t sc0, mn0, sc1, mn1;
        q4_scale_min(hd[i].y, hd[i].z, hd[i].w, g, sc0, mn0, sc1, mn1);
        const float d = h2f(hd[i].x & 0xFFFF), dmin = h2f(hd[i].x >> 16);
        const uint32_t qw[8] = {q0[i].x, q0[i].y, q0[i].z, q0[i].w, q1[i].x, q1[i].y, q1[i].z, q1[i].w};
        float S0 = 0.0f, S1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // bytes 0-15: pair 0
            uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
            hide_bits(lo), hide_bits(hi);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S0 = fmaf((float)((lo >> (8 * e)) & 0xFF), xv[4 * k + e], S0);
                S0 = fmaf((float)((hi >> (8 * e)) & 0xFF), xv[32 + 4 * k + e], S0);
            }
        }
#pragma unroll
        for (int k = 4; k < 8; ++k) {  // bytes 16-31: pair 1
            uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
            hide_bits(lo), hide_bits(hi);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S1 = fmaf((float)((lo >> (8 * e)) & 0xFF), xv[4 * k + e], S1);
                S1 = fmaf((float)((hi >> (8 * e)) & 0xFF), xv[32 + 4 * k + e], S1);
            }
        }
        const float val = ((d * (float)sc0) * S0 + (d * (float)sc1) * S1) -
                          dmin * ((float)mn0 * xm.x + (float)mn1 * xm.y);
        red[ph0 < P ? rr * nq + q : R * nq] = val;  // padding threads: the spare slot
    }
    __syncthreads();
    row_sums_store(red, nq, nr, G, yp, y, r0);
}

template <int RPT>
int launch_q4_f32_x(uint32_t xpt, dim3 grid, dim3 blk, size_t lds, hipStream_t st, const uint8_t* W, const float* x,
                    float* y, uint32_t M, uint32_t nsb, uint32_t P, uint32_t R, uint32_t G, uint32_t mg) {
    switch (xpt) {
        case 1: hipLaunchKernelGGL((k_gguf_q4_K_f32<RPT, 1>), grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg); break;
        case 2: hipLaunchKernelGGL((k_gguf_q4_K_f32<RPT, 2>), grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg); break;
        case 4: hipLaunchKernelGGL((k_gguf_q4_K_f32<RPT, 4>), grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg); break;
        case 8: hipLaunchKernelGGL((k_gguf_q4_K_f32<RPT, 8>), grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg); break;
        case 16: hipLaunchKernelGGL((k_gguf_q4_K_f32<RPT, 16>), grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg); break;
        default: return EC_ERR_UNSUPPORTED;
    }
    return EC_OK;
}

int launch_q4_f32(uint32_t rpt, uint32_t xpt, dim3 grid, dim3 blk, size_t lds, hipStream_t st, const uint8_t* W,
                  const float* x, float* y, uint32_t M, uint32_t nsb, uint32_t P, uint32_t R) {
    const uint32_t nq = 4 * nsb, mg = (uint32_t)((((uint64_t)1 << 32) + nq - 1) / nq);
    uint32_t G = 64;  // threads per row in the row sums: a power of two with G * R <= T
    while (G * R > blk.x) G /= 2;
    if (rpt == 4) return launch_q4_f32_x<4>(xpt, grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg);
    if (rpt == 2) return launch_q4_f32_x<2>(xpt, grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg);
    return launch_q4_f32_x<1>(xpt, grid, blk, lds, st, W, x, y, M, nsb, P, R, G, mg);
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
    static const uint32_t rpt_env = [] {
        const char* v = getenv("EC_GGUF_RPT");  // 1, 2 or 4: fixed rows per thread, for comparison
        return v ? (uint32_t)atoi(v) : 0u;
    }();
    if (fmt == EC_Q8_0) {
        if (K % 64 || K / 64 > 1024) return EC_ERR_UNSUPPORTED;
        const uint32_t nc = K / 64;  // block pairs per row
        // Four threads per pair column (at least one wave per workgroup, at
        // most 1024 threads), one row per thread, two where one would mean
        // more than 4096 workgroups.  Swept over 12 shapes (P = 1 .. 16,
        // 1 / 2 / 4 rows per thread; graph-timed us): this choice is within
        // 5% of each shape's best -- 9216 x 2560 7.89 (best 7.67), 2560 x 9216
        // 9.07, 12352 x 2560 9.24, 2560 x 4096 5.42, 6144 x 2560 6.35, 18432 x
        // 2560 12.43 (two rows; one row 13.39), 4096 x 11008 13.53, 1024 x 2560
        // 3.49 -- and four rows per thread, which leave few workgroups, were
        // never the best (1024 x 2560: 9.8).
        uint32_t P = 4;
        while (P * nc < 64) P *= 2;
        while (P > 1 && P * nc > 1024) P /= 2;
        static const uint32_t q8p_env = [] {
            const char* v = getenv("EC_GGUF_Q8_P");  // threads per pair column (a power of two), for comparison
            return v ? (uint32_t)atoi(v) : 0u;
        }();
        if (q8p_env && (q8p_env & (q8p_env - 1)) == 0 && q8p_env * nc <= 1024) P = q8p_env;
        const uint32_t T = (P * nc + 63) / 64 * 64;
        uint32_t rpt = (M + P - 1) / P > 4096 ? 2 : 1;
        if (rpt_env == 1 || rpt_env == 2) rpt = rpt_env;
        const uint32_t R = rpt * P;
        uint32_t xpt = 1;
        while (xpt * T < 16 * nc) xpt *= 2;
        uint32_t G = 64;  // threads per row in the row sums: a power of two with G * R <= T
        while (G * R > T) G /= 2;
        const size_t lds = q8_f32_lds_bytes(nc, R);
        const uint32_t mg = (uint32_t)((((uint64_t)1 << 32) + nc - 1) / nc);
        if (xpt > 16 || G < 1 || lds > 160 * 1024) return EC_ERR_UNSUPPORTED;  // gfx950: 160 KB per workgroup
        const dim3 grid((M + R - 1) / R), blk(T);
        if (rpt == 2) return launch_q8_f32_x<2>(xpt, grid, blk, lds, st, W, x, y, M, nc, P, R, G, mg);
        return launch_q8_f32_x<1>(xpt, grid, blk, lds, st, W, x, y, M, nc, P, R, G, mg);
    }
    if (fmt == EC_Q4_K) {
        const uint32_t nsb = K / 256, nq = 4 * nsb;
        if (nq > 1024) return EC_ERR_UNSUPPORTED;
        // threads per quarter: the smallest power of two that makes P * nq a
        // whole number of waves and at least 256 threads (2560 x 4096, nq =
        // 64: one thread per quarter 7.7 us, four 4.55 us; more threads than
        // that were no faster at K = 2560, 4096 or 9216)
        uint32_t P = 64 / gcd32(nq, 64);
        while (P * nq < 256 && 2 * P * nq <= 1024) P *= 2;
        while (P > 1 && P * nq > 1024) P /= 2;
        static const uint32_t p_env = [] {
            const char* v = getenv("EC_GGUF_P");  // threads per quarter (a power of two), for comparison
            return v ? (uint32_t)atoi(v) : 0u;
        }();
        if (p_env && (p_env & (p_env - 1)) == 0 && p_env * nq <= 1024) P = p_env;
        // RPT rows per thread (all rows' loads in flight): x is read from L2
        // once per workgroup of R = RPT * P rows, so larger R means fewer
        // activation bytes per weight byte, but fewer waves to hide the
        // latency and spread the arithmetic; RPT = 1 while that leaves at
        // least 512 workgroups, else 2, else 4
        uint32_t rpt = 1;
        while (rpt < 4 && (M + rpt * P - 1) / (rpt * P) < 512) rpt *= 2;
        const uint32_t T = (P * nq + 63) / 64 * 64;
        if (rpt == 4 && T > (uint32_t)q4_f32_max_threads<4>()) rpt = 2;
        if ((rpt_env == 1 || rpt_env == 2 || rpt_env == 4) && T <= (rpt_env == 4 ? 768u : 1024u)) rpt = rpt_env;
        const uint32_t R = rpt * P;
        const dim3 grid((M + R - 1) / R), blk(T);
        const size_t lds = q4_f32_lds_bytes(nq, R);
        // x's 16 * nq float4s over T threads, rounded up to a compiled count
        uint32_t xpt = 1;
        while (xpt * T < 16 * nq) xpt *= 2;
        if (T > 1024 || R > T || lds > 160 * 1024 || xpt > 16) return EC_ERR_UNSUPPORTED;
        return launch_q4_f32(rpt, xpt, grid, blk, lds, st, W, x, y, M, nsb, P, R);
    }
    return EC_ERR_UNSUPPORTED;
}

}  // namespace ec
