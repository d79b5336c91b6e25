// quant.hip — quantizers, weight repacking and activation packing (gfx950).
//
// Layouts (all byte offsets little-endian):
//
// Q8_0 tiled weights ("Q8T"): rows in tiles of 16, K in groups of 4 blocks
// (128 elements).  Chunk (tile t, group G) = 2176 bytes at (t*nG+G)*2176:
//   [0,1024)    lane l (0..63) owns bytes [16l, 16l+16): for j=0..1 the 8 int8
//               weights W[16t + l%16][128G + 32j + 8(l/16) .. +8]
//   [1024,2048) the same for j=2..3 at 1024 + 16l
//   [2048,2176) row r (0..15) owns 8 bytes: fp16 d of blocks 4G..4G+3
// Lane l's 8 bytes per block are exactly its B operand of
// v_mfma_i32_16x16x32_i8 (B[k][j]: lane j + 16*(k/8), byte k%8), so a wave
// streams 2 KB of weights with two 16-byte loads per lane, each load
// instruction covering one contiguous 1 KB, and no shuffles.
//
// Q4_K tiled weights ("Q4T"): chunk (tile t, super-block b) = 2304 bytes:
//   [0,1024)   lane l owns bytes [16l, 16l+16): for sub-block s=0..3 the 4
//              packed bytes qs[16s + 4g .. +4] (g = l/16) of row 16t + l%16
//   [1024,2048) the same for s=4..7 at 1024 + 16l
//   [2048,2304) row r owns its 16-byte header (d, dmin, scales[12])
// With k' = 8g + j, j<4 -> low nibble of byte 4g+j, j>=4 -> high nibble of
// byte 4g+j-4, the MFMA k index of sub-block s maps to element
// e = 4g+j (j<4) or 16+4g+j-4 (j>=4) of the sub-block (oc_q4k_pos order).
//
// Activations ("act") for M <= 16 token rows, per format:
//   xq   Q8_0: [nG][4][M][32 B]: j=0..3 x 8 int8 of x[i][128G+32j+8g..+8]
//        Q4_K: [nB][4][M][64 B]: s=0..7 x (xsub[4g..+4], xsub[16+4g..+4])
//   xd   fp32 [16][Kp/32]   scale of each 32-block per token slot (0 for padding)
//   dxs  fp32 [16][Kp/32]   Q4_K only: xd * sum(block int8), the min term
// Two-piece activations (P = 2) store M tokens as 2M rows of xq, token i's
// piece p (q_piece1 for p = 1, scale xd/256) in row 2i + p, with xd and dxs
// per token as above (dxs = xd * (sum q0 + sum q1 / 256)).
#include "common.hpp"
#include "layout.hpp"

namespace ec {

// ------------------------------------------------------------ row quantizer
// One wave per row.  The reference's body/tail split is by element index.
__global__ __launch_bounds__(64) void k_quantize_rows(const float* __restrict__ x, int8_t* __restrict__ q,
                                                      float* __restrict__ scales, uint32_t rows, uint32_t width) {
    uint32_t r = blockIdx.x;
    if (r >= rows) return;
    const float* xr = x + (size_t)r * width;
    int8_t* qr = q + (size_t)r * width;
    float amax = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += 64) amax = fmaxf(amax, fabsf(xr[i]));
    amax = wave_max(amax);
    float scale = q_scale(amax);
    float inv = __fdiv_rn(1.0f, scale);
    uint32_t body = width & ~7u;
    for (uint32_t i = threadIdx.x; i < width; i += 64) qr[i] = (i < body) ? q_body(xr[i], inv) : q_tail(xr[i], scale);
    if (threadIdx.x == 0) scales[r] = scale;
}

// ------------------------------------------------------------------ repack
// One thread per (row, block) of the padded grid.
__global__ void k_repack_q8_0(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t N, uint32_t K,
                              uint32_t Np, uint32_t Kp) {
    uint32_t nbp = Kp / 32, nb = K / 32;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)Np * nbp) return;
    uint32_t row = idx / nbp, b = idx % nbp;
    uint8_t blk[34];
    if (row < N && b < nb) {
        const uint8_t* s = src + ((size_t)row * nb + b) * 34;
        for (int i = 0; i < 34; ++i) blk[i] = s[i];
    } else {
        for (int i = 0; i < 34; ++i) blk[i] = 0;
    }
    uint32_t nG = Kp / 128, t = row / 16, r = row % 16, G = b / 4, j = b % 4;
    uint8_t* ch = dst + ((size_t)t * nG + G) * 2176;
    for (int g = 0; g < 4; ++g) {
        uint8_t* p = ch + (j / 2) * 1024 + (size_t)(r + 16 * g) * 16 + 8 * (j % 2);
        for (int e = 0; e < 8; ++e) p[e] = blk[2 + 8 * g + e];
    }
    ch[2048 + r * 8 + 2 * j] = blk[0];
    ch[2048 + r * 8 + 2 * j + 1] = blk[1];
}

__global__ void k_repack_q4_K(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t N, uint32_t K,
                              uint32_t Np, uint32_t Kp) {
    uint32_t nbp = Kp / 256, nb = K / 256;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)Np * nbp) return;
    uint32_t row = idx / nbp, b = idx % nbp;
    const uint8_t* s = (row < N && b < nb) ? src + ((size_t)row * nb + b) * 144 : nullptr;
    uint32_t t = row / 16, r = row % 16;
    uint8_t* ch = dst + ((size_t)t * nbp + b) * 2304;
    for (int i = 0; i < 16; ++i) ch[2048 + r * 16 + i] = s ? s[i] : 0;
    for (int g = 0; g < 4; ++g)
        for (int sb = 0; sb < 8; ++sb)
            for (int e = 0; e < 4; ++e)
                ch[(sb / 4) * 1024 + (size_t)(r + 16 * g) * 16 + 4 * (sb % 4) + e] = s ? s[16 + 16 * sb + 4 * g + e] : 0;
}

// Inverse of k_repack_q8_0: tiled -> GGUF rows (only the N x K/32 real blocks).
__global__ void k_unpack_q8_0(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t N, uint32_t K,
                              uint32_t Kp) {
    const uint32_t nb = K / 32;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * nb) return;
    const uint32_t row = idx / nb, b = idx % nb;
    const uint32_t nG = Kp / 128, t = row / 16, r = row % 16, G = b / 4, j = b % 4;
    const uint8_t* ch = src + ((size_t)t * nG + G) * 2176;
    uint8_t* o = dst + ((size_t)row * nb + b) * 34;
    o[0] = ch[2048 + r * 8 + 2 * j];
    o[1] = ch[2048 + r * 8 + 2 * j + 1];
    for (int g = 0; g < 4; ++g) {
        const uint8_t* p = ch + (j / 2) * 1024 + (size_t)(r + 16 * g) * 16 + 8 * (j % 2);
        for (int e = 0; e < 8; ++e) o[2 + 8 * g + e] = p[e];
    }
}

// Inverse of k_repack_q4_K: tiled -> GGUF rows (only the N x K/256 real super-blocks).
__global__ void k_unpack_q4_K(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t N, uint32_t K,
                              uint32_t Kp) {
    const uint32_t nb = K / 256, nbp = Kp / 256;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * nb) return;
    const uint32_t row = idx / nb, b = idx % nb, t = row / 16, r = row % 16;
    const uint8_t* ch = src + ((size_t)t * nbp + b) * 2304;
    uint8_t* o = dst + ((size_t)row * nb + b) * 144;
    for (int i = 0; i < 16; ++i) o[i] = ch[2048 + r * 16 + i];
    for (int g = 0; g < 4; ++g)
        for (int sb = 0; sb < 8; ++sb)
            for (int e = 0; e < 4; ++e)
                o[16 + 16 * sb + 4 * g + e] = ch[(sb / 4) * 1024 + (size_t)(r + 16 * g) * 16 + 4 * (sb % 4) + e];
}

// ------------------------------------------------------- activation packing
// One thread per (token slot i < 16, 32-block).  Slots >= M only zero scales.
__global__ void k_quantize_act_q8_0(const float* __restrict__ x, uint8_t* __restrict__ act, uint32_t M, uint32_t K,
                                    uint32_t Kp, size_t xd_off, uint32_t P) {
    uint32_t nbp = Kp / 32;
    uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 16 * nbp) return;
    uint32_t i = idx % 16, sb = idx / 16;
    float* xd = (float*)(act + xd_off);
    if (i >= M) {
        xd[(size_t)i * nbp + sb] = 0.0f;
        return;
    }
    float v[32];
    bool real = sb < K / 32;
    float amax = 0.0f;
    for (int e = 0; e < 32; ++e) {
        v[e] = real ? x[(size_t)i * K + 32 * sb + e] : 0.0f;
        amax = fmaxf(amax, fabsf(v[e]));
    }
    float scale = real ? q_scale(amax) : 0.0f;
    float inv = real ? __fdiv_rn(1.0f, scale) : 0.0f;
    int8_t qv[32];
    for (int e = 0; e < 32; ++e) qv[e] = real ? q_body(v[e], inv) : 0;
    uint32_t G = sb / 4, j = sb % 4;
    for (int g = 0; g < 4; ++g) {
        uint8_t* p = act + (((size_t)G * 4 + g) * (P * M) + P * i) * 32 + 8 * j;
        for (int e = 0; e < 8; ++e) p[e] = (uint8_t)qv[8 * g + e];
        if (P == 2)
            for (int e = 0; e < 8; ++e)
                p[32 + e] = real ? (uint8_t)q_piece1(v[8 * g + e], qv[8 * g + e], scale, inv) : (uint8_t)0;
    }
    xd[(size_t)i * nbp + sb] = scale;
}

__global__ void k_quantize_act_q4_K(const float* __restrict__ x, uint8_t* __restrict__ act, uint32_t M, uint32_t K,
                                    uint32_t Kp, size_t xd_off, size_t dxs_off, uint32_t P) {
    uint32_t nsb = Kp / 32;
    uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 16 * nsb) return;
    uint32_t i = idx % 16, sbi = idx / 16;
    float* xd = (float*)(act + xd_off);
    float* dxs = (float*)(act + dxs_off);
    if (i >= M) {
        xd[(size_t)i * nsb + sbi] = 0.0f;
        dxs[(size_t)i * nsb + sbi] = 0.0f;
        return;
    }
    uint32_t b = sbi / 8, s = sbi % 8, gq = s / 2, p = s % 2;
    bool real = b < K / 256;
    size_t base = (size_t)i * K + 256 * (size_t)b + 64 * gq + 16 * p;
    float v[32];
    float amax = 0.0f;
    for (int e = 0; e < 16; ++e) {
        v[e] = real ? x[base + e] : 0.0f;
        v[16 + e] = real ? x[base + 32 + e] : 0.0f;
    }
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
    float scale = real ? q_scale(amax) : 0.0f;
    float inv = real ? __fdiv_rn(1.0f, scale) : 0.0f;
    int8_t qv[32], qv1[32];
    int sum = 0, sum1 = 0;
    for (int e = 0; e < 32; ++e) {
        qv[e] = real ? q_body(v[e], inv) : 0;
        qv1[e] = (real && P == 2) ? q_piece1(v[e], qv[e], scale, inv) : 0;
        sum += qv[e];
        sum1 += qv1[e];
    }
    for (int g = 0; g < 4; ++g) {
        uint8_t* dp = act + (((size_t)b * 4 + g) * (P * M) + P * i) * 64 + 8 * s;
        for (int e = 0; e < 4; ++e) {
            dp[e] = (uint8_t)qv[4 * g + e];
            dp[4 + e] = (uint8_t)qv[16 + 4 * g + e];
        }
        if (P == 2)
            for (int e = 0; e < 4; ++e) {
                dp[64 + e] = (uint8_t)qv1[4 * g + e];
                dp[64 + 4 + e] = (uint8_t)qv1[16 + 4 * g + e];
            }
    }
    xd[(size_t)i * nsb + sbi] = scale;
    // the min term's activation sum: scale * sum(q0), or with two pieces
    // (scale/256) * (256 sum(q0) + sum(q1)), the integer sum exact
    dxs[(size_t)i * nsb + sbi] =
        P == 2 ? __fmul_rn(scale * (1.0f / 256.0f), (float)(256 * sum + sum1)) : __fmul_rn(scale, (float)sum);
}

// One thread per (layout row i < R = P*M, block); row i's bytes to xq[i], and
// for piece-0 rows the token's scale to xdo[i / P].
__global__ void k_act_unpack(int fmt, const uint8_t* __restrict__ act, int8_t* __restrict__ xq,
                             float* __restrict__ xdo, uint32_t R, uint32_t K, uint32_t Kp, size_t xd_off,
                             uint32_t P) {
    uint32_t nb = K / 32;
    uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= R * nb) return;
    uint32_t i = idx / nb, sb = idx % nb;
    const uint32_t M = R;  // layout rows
    const float* xd = (const float*)(act + xd_off);
    int8_t* out = xq + (size_t)i * K + 32 * sb;
    if (fmt == EC_Q8_0) {
        uint32_t G = sb / 4, j = sb % 4;
        for (int g = 0; g < 4; ++g)
            for (int e = 0; e < 8; ++e) out[8 * g + e] = (int8_t)act[(((size_t)G * 4 + g) * M + i) * 32 + 8 * j + e];
    } else {
        uint32_t b = sb / 8, s = sb % 8;
        for (int g = 0; g < 4; ++g)
            for (int e = 0; e < 4; ++e) {
                out[4 * g + e] = (int8_t)act[(((size_t)b * 4 + g) * M + i) * 64 + 8 * s + e];
                out[16 + 4 * g + e] = (int8_t)act[(((size_t)b * 4 + g) * M + i) * 64 + 8 * s + 4 + e];
            }
    }
    if (i % P == 0) xdo[(size_t)(i / P) * nb + sb] = xd[(size_t)(i / P) * (Kp / 32) + sb];
}

// ------------------------------------------------------------------ random
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ double u01(uint64_t z) { return (double)(z >> 40) * (1.0 / 16777216.0); }
__device__ __forceinline__ double normal_at(uint64_t seed, uint64_t i) {
    double u1 = 1.0 - u01(splitmix64_at(seed, 2 * i));
    double u2 = u01(splitmix64_at(seed, 2 * i + 1));
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

// kind 0: bytes; kind 1: Q8_0 GGUF blocks (n = number of blocks); kind 2: fp32 normals.
// Seeds follow echohip/synth.py: stream s seed = splitmix64_at(seed, s).
__global__ void k_fill_random(int kind, uint8_t* dst, uint64_t n, uint64_t seed, float scale) {
    uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    if (kind == 0) {
        for (; idx < n; idx += stride) dst[idx] = (uint8_t)splitmix64_at(seed, idx);
    } else if (kind == 1) {
        uint64_t s0 = splitmix64_at(seed, 0), s1 = splitmix64_at(seed, 1);
        for (; idx < n; idx += stride) {
            uint8_t* blk = dst + idx * 34;
            float d = (float)(fabs(normal_at(s1, idx)) * (double)scale);
            uint16_t h = __half_as_ushort(__float2half_rn(d));
            blk[0] = h & 0xFF;
            blk[1] = h >> 8;
            for (int j = 0; j < 32; ++j) {
                int64_t q = (int64_t)(splitmix64_at(s0, idx * 32 + j) % 255ull) - 127;
                blk[2 + j] = (uint8_t)(int8_t)q;
            }
        }
    } else {
        float* f = (float*)dst;
        for (; idx < n; idx += stride) f[idx] = (float)(normal_at(seed, idx) * (double)scale);
    }
}

}  // namespace ec

// ======================================================================== C ABI
using namespace ec;

static thread_local char g_err[512] = "";

extern "C" const char* ec_last_error(void) { return g_err; }

extern "C" void ec_clear_error(void) { g_err[0] = 0; }

extern "C" int ec_set_error(int code, const char* msg) {
    snprintf(g_err, sizeof(g_err), "%s", msg);
    return code;
}

extern "C" int ec_set_hip_error(hipError_t e, const char* where) {
    snprintf(g_err, sizeof(g_err), "%s: %s", where, hipGetErrorString(e));
    return EC_ERR_HIP;
}

extern "C" int ec_attn_scratch_init(int device);

extern "C" int ec_device_init(int device) {
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return ec_set_hip_error(e, "ec_device_init");
    return ec_attn_scratch_init(device);  // the device address of ec_attn_decode_noalloc's scratch
}

extern "C" int ec_copy(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return EC_OK;
    if (!dst || !src) return ec_set_error(EC_ERR_ARG, "ec_copy: null pointer");
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDefault);
    if (e != hipSuccess) return ec_set_hip_error(e, "ec_copy");
    return EC_OK;
}

extern "C" int ec_quantize_rows(const float* x, int8_t* q, float* scales, uint32_t rows, uint32_t width,
                                void* stream) {
    if (rows == 0) return EC_OK;
    if (!x || !q || !scales || width == 0) return ec_set_error(EC_ERR_ARG, "ec_quantize_rows: bad argument");
    hipLaunchKernelGGL(k_quantize_rows, dim3(rows), dim3(64), 0, (hipStream_t)stream, x, q, scales, rows, width);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" size_t ec_tiled_bytes(int fmt, uint32_t N, uint32_t K) {
    uint32_t Np = round_up(N, 16);
    if (fmt == EC_Q8_0) return (size_t)(Np / 16) * (round_up(K, 128) / 128) * 2176;
    if (fmt == EC_Q4_K) return (size_t)(Np / 16) * (round_up(K, 256) / 256) * 2304;
    return 0;
}

extern "C" int ec_repack(int fmt, const void* gguf, void* tiled, uint32_t N, uint32_t K, void* stream) {
    if (!gguf || !tiled || N == 0) return ec_set_error(EC_ERR_ARG, "ec_repack: bad argument");
    uint32_t Np = round_up(N, 16);
    if (fmt == EC_Q8_0) {
        if (K % 32) return ec_set_error(EC_ERR_ARG, "ec_repack: Q8_0 needs K % 32 == 0");
        uint32_t Kp = round_up(K, 128);
        size_t n = (size_t)Np * (Kp / 32);
        hipLaunchKernelGGL(k_repack_q8_0, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           (const uint8_t*)gguf, (uint8_t*)tiled, N, K, Np, Kp);
    } else if (fmt == EC_Q4_K) {
        if (K % 256) return ec_set_error(EC_ERR_ARG, "ec_repack: Q4_K needs K % 256 == 0");
        uint32_t Kp = round_up(K, 256);
        size_t n = (size_t)Np * (Kp / 256);
        hipLaunchKernelGGL(k_repack_q4_K, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           (const uint8_t*)gguf, (uint8_t*)tiled, N, K, Np, Kp);
    } else {
        return ec_set_error(EC_ERR_UNSUPPORTED, "ec_repack: format must be Q8_0 or Q4_K");
    }
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_unpack_tiled(int fmt, const void* tiled, void* gguf, uint32_t N, uint32_t K, void* stream) {
    if (fmt == EC_Q4_K) {
        if (!tiled || !gguf || K % 256) return ec_set_error(EC_ERR_ARG, "ec_unpack_tiled: bad argument");
        const size_t n = (size_t)N * (K / 256);
        if (n == 0) return EC_OK;
        hipLaunchKernelGGL(k_unpack_q4_K, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           (const uint8_t*)tiled, (uint8_t*)gguf, N, K, round_up(K, 256));
        EC_CHECK_LAUNCH();
        return EC_OK;
    }
    if (fmt != EC_Q8_0) return ec_set_error(EC_ERR_UNSUPPORTED, "ec_unpack_tiled: Q8_0 or Q4_K");
    if (!tiled || !gguf || K % 32) return ec_set_error(EC_ERR_ARG, "ec_unpack_tiled: bad argument");
    const size_t n = (size_t)N * (K / 32);
    if (n == 0) return EC_OK;
    hipLaunchKernelGGL(k_unpack_q8_0, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)tiled, (uint8_t*)gguf, N, K, round_up(K, 128));
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" size_t ec_act_bytes(int fmt, uint32_t M, uint32_t K) {
    if (fmt != EC_Q8_0 && fmt != EC_Q4_K) return 0;
    return act_layout(fmt, M, K).total;
}

extern "C" size_t ec_act_bytes_pieces(int fmt, uint32_t M, uint32_t K, uint32_t pieces) {
    if ((fmt != EC_Q8_0 && fmt != EC_Q4_K) || (pieces != 1 && pieces != 2)) return 0;
    return act_layout(fmt, pieces * M, K).total;
}

extern "C" int ec_quantize_act_pieces(int fmt, const float* x, void* act, uint32_t M, uint32_t K, uint32_t pieces,
                                      void* stream) {
    if (!x || !act || M == 0 || M > 16 || K == 0 || K % 32 || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_quantize_act: need 1 <= M <= 16, K % 32 == 0, 1 or 2 pieces");
    ActLayout L = act_layout(fmt, pieces * M, K);
    uint32_t n = 16 * (L.Kp / 32);
    if (fmt == EC_Q8_0) {
        hipLaunchKernelGGL(k_quantize_act_q8_0, dim3((n + 127) / 128), dim3(128), 0, (hipStream_t)stream, x,
                           (uint8_t*)act, M, K, L.Kp, L.xd_off, pieces);
    } else if (fmt == EC_Q4_K) {
        if (K % 256) return ec_set_error(EC_ERR_ARG, "ec_quantize_act: Q4_K needs K % 256 == 0");
        hipLaunchKernelGGL(k_quantize_act_q4_K, dim3((n + 127) / 128), dim3(128), 0, (hipStream_t)stream, x,
                           (uint8_t*)act, M, K, L.Kp, L.xd_off, L.dxs_off, pieces);
    } else {
        return ec_set_error(EC_ERR_UNSUPPORTED, "ec_quantize_act: format must be Q8_0 or Q4_K");
    }
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_quantize_act(int fmt, const float* x, void* act, uint32_t M, uint32_t K, void* stream) {
    return ec_quantize_act_pieces(fmt, x, act, M, K, 1, stream);
}

extern "C" int ec_act_unpack_pieces(int fmt, uint32_t pieces, const void* act, int8_t* xq, float* xd, uint32_t M,
                                    uint32_t K, void* stream) {
    if (!act || !xq || !xd || M == 0 || M > 16 || K % 32 || (fmt != EC_Q8_0 && fmt != EC_Q4_K) ||
        (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_act_unpack: bad argument");
    ActLayout L = act_layout(fmt, pieces * M, K);
    uint32_t n = pieces * M * (K / 32);
    hipLaunchKernelGGL(k_act_unpack, dim3((n + 127) / 128), dim3(128), 0, (hipStream_t)stream, fmt,
                       (const uint8_t*)act, xq, xd, pieces * M, K, L.Kp, L.xd_off, pieces);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_act_unpack(int fmt, const void* act, int8_t* xq, float* xd, uint32_t M, uint32_t K, void* stream) {
    return ec_act_unpack_pieces(fmt, 1, act, xq, xd, M, K, stream);
}

extern "C" int ec_fill_random(int kind, void* dst, uint64_t n, uint64_t seed, float scale, uint32_t K,
                              void* stream) {
    (void)K;
    if (!dst || kind < 0 || kind > 2) return ec_set_error(EC_ERR_ARG, "ec_fill_random: bad argument");
    if (n == 0) return EC_OK;
    hipLaunchKernelGGL(k_fill_random, dim3(4096), dim3(256), 0, (hipStream_t)stream, kind, (uint8_t*)dst, n, seed,
                       scale);
    EC_CHECK_LAUNCH();
    return EC_OK;
}
