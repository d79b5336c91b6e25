// matvec.hip — decode matvec / skinny GEMM over block-quantized weights.
//
// y[m][n] (+)= sum over 32-element blocks of d_w * d_x * isum for M <= 16 token
// rows (src/kernels/matvec.cpp:62-142 computes the same sums for one row of
// fp32 activations).  The integer block dot isum is one
// v_mfma_i32_16x16x32_i8: A = 16 token rows x 32 int8 activations, B = 32 int8
// weights x 16 weight rows, so a wave turns 16 rows x 32 elements of weights
// into 16x16 exact int32 dots per instruction.  The kernel is a weight stream:
// each wave reads a contiguous run of 2 KB chunks of the tiled layout (two
// 16-byte loads per lane per chunk, each instruction one contiguous 1 KB),
// the 16-token activation operand comes
// from L1/L2, and the fp32 epilogue applies the per-block scales.  The K range
// of one 16-row tile is split across the waves of a workgroup and reduced
// through LDS in a fixed order (deterministic results).
//
// MFMA lane layout (16x16x32 i8): A[i][k] and B[k][j] live in lane
// (i or j) + 16*(k/8), byte k%8; D[i][j] lives in lane j + 16*(i/4), element i%4.
//
// Two-piece activations (P = 2): token i's pieces are A rows 2i and 2i+1
// (rows 16a.. of MFMA group a for tokens 8a..), so D rows 2i and 2i+1 sit in
// one lane and the epilogue combines them exactly as 256*dot0 + dot1 (|dot| <=
// 2^19: no int32 overflow), one conversion and one FMA with d_w * d_x / 256.
#include "common.hpp"
#include "layout.hpp"
#include <cstring>

namespace ec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Weight loads are streaming (each byte is used once per step): non-temporal.
__device__ __forceinline__ uint4 ld_stream16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream8(const uint8_t* p) {
    const u32x2 v = __builtin_nontemporal_load((const u32x2*)p);
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

__device__ __forceinline__ v4i mfma_i8(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// Output token of accumulator r of a lane in D row group g: P = 1, token
// 4g + r (D row = token); P = 2, token 8(r/2) + 2g + r%2 (MFMA group r/2).
template <int P>
__device__ __forceinline__ uint32_t out_token(uint32_t g, uint32_t r) {
    return P == 1 ? 4 * g + r : 8 * (r >> 1) + 2 * g + (r & 1);
}

// Cross-wave reduction of the TPW tiles' acc[4] and the store of y /
// accumulate.  Each wave parks its partials in LDS (red: [TPW][waves][R][64]);
// then thread q (q < TPW*R*64) sums accumulator r of lane l of tile tt over
// the waves in wave order (deterministic) and stores it: weight row
// 16(t0 + tt) + l%16, token out_token(l/16, r).  Measured on the batch-8
// decode step's 128 projections: 999 -> 990 us per step against a [..][lane][4]
// layout (8-way LDS bank conflicts) summed one wave per LDS round trip.
template <int R, int P, int TPW>
__device__ __forceinline__ void reduce_store(float (&acc)[TPW][4], float* red, float* __restrict__ y, uint32_t t0,
                                             uint32_t M, uint32_t N, uint32_t ldy, int accumulate) {
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (nw == 1) {
        const uint32_t row = lane & 15, g = lane >> 4;
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const uint32_t n = 16 * (t0 + tt) + row;
            if (n >= N) continue;
            for (int r = 0; r < R; ++r) {
                const uint32_t m = out_token<P>(g, r);
                if (m < M) {
                    float* dst = y + (size_t)m * ldy + n;
                    *dst = accumulate ? *dst + acc[tt][r] : acc[tt][r];
                }
            }
        }
        return;
    }
    // red[tt][w][r][lane]: consecutive lanes touch consecutive dwords (no
    // LDS bank conflicts on the writes or on the reads below)
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
        for (int r = 0; r < R; ++r) red[((tt * nw + w) * R + r) * 64 + lane] = acc[tt][r];
    __syncthreads();
    // thread q: tile q / (64R), accumulator (q / 64) % R of lane q % 64.  The
    // waves' values are summed in wave order; their LDS reads are issued
    // eight at a time (clamped to the last wave), not one round trip per wave:
    // this sum is the tail of the workgroup, and of the launch.
    for (uint32_t q = threadIdx.x; q < 64 * R * TPW; q += blockDim.x) {
        const uint32_t ln = q & 63, r = (q >> 6) % R, tt = (q >> 6) / R;
        const uint32_t m = out_token<P>(ln >> 4, r), n = 16 * (t0 + tt) + (ln & 15);
        if (m >= M || n >= N) continue;
        const float* rs = red + ((size_t)tt * nw * R + r) * 64 + ln;
        float s = rs[0];
        for (uint32_t v0 = 1; v0 < nw; v0 += 8) {
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = rs[min(v0 + i, nw - 1) * (64 * R)];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (v0 + i < nw) s += x[i];
        }
        float* dst = y + (size_t)m * ldy + n;
        *dst = accumulate ? *dst + s : s;
    }
}

// ------------------------------------------------------------ wave program
// Every wave owns GPW consecutive chunks (2 KB Q8_0 groups or 2.3 KB Q4_K
// super-blocks) of one 16-row tile and runs straight-line code:
//   1. load the activation scales of its blocks (vector loads, issued first),
//   2. load all GPW weight chunks and activation operands (no branches: an
//      index past the wave's range is clamped, the chunk is loaded again and
//      not computed; an empty token slot reads token 0 and is zeroed at use),
//   3. stage the scales in the wave's own LDS slice (waits only for step 1),
//   4. MFMA + fp32 epilogue chunk by chunk as the loads land.
// With no data-dependent branch around a load, the compiler's waitcnts count
// exactly and GPW*2 KB per wave stay in flight.
template <int MT>
constexpr int slots() { return MT == 1 ? 1 : (MT <= 4 ? 4 : (MT <= 8 ? 8 : 16)); }
// Activation layout rows staged per token slot group: P pieces per token.
template <int MT, int P>
constexpr int lrows() { return P * slots<MT>(); }
// MFMA row groups (16 layout rows each) and accumulators per lane.
template <int MT, int P>
constexpr int ngroups() { return (lrows<MT, P>() + 15) / 16; }
template <int MT, int P>
constexpr int naccs() { return P == 1 ? (MT < 4 ? MT : 4) : (MT == 1 ? 1 : 2 * ngroups<MT, P>()); }

// Scales of blocks [b0, b0+NB) for token slots [0, S): LDS slice xs[NB][S],
// source layout token-major [16][nblk].  Values for tokens >= M are zero;
// PRE multiplies every value by 1/256 (the two-piece epilogue's step).
template <int NB, int S, bool PRE = false>
struct ScaleStage {
    static constexpr int N = NB * S;
    static constexpr int PER_LANE = (N + 63) / 64;
    float v[PER_LANE];
    __device__ __forceinline__ void load(const float* __restrict__ src, uint32_t nblk, uint32_t b0, uint32_t M,
                                         uint32_t lane) {
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i) {
            const uint32_t e = lane + 64 * i;
            const uint32_t b = b0 + e / S, t = e % S;
            const bool ok = e < (uint32_t)N && b < nblk && t < M;
            const float x = src[(size_t)(ok ? t : 0) * nblk + (ok ? b : 0)];
            v[i] = ok ? (PRE ? x * (1.0f / 256.0f) : x) : 0.0f;
        }
    }
    __device__ __forceinline__ void store(float* xs, uint32_t lane) const {
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i) {
            const uint32_t e = lane + 64 * i;
            if (e < (uint32_t)N) xs[e] = v[i];
        }
    }
};

// A wave's activation operand bytes for its chunks form one contiguous range
// (the act layout is chunk-major); it is loaded with full 1 KB-per-instruction
// loads, clamped to the buffer, and staged in LDS next to the scales.
template <int MAXB>
struct ByteStage {
    static constexpr int PER_LANE = (MAXB + 1023) / 1024;
    uint4 v[PER_LANE];
    __device__ __forceinline__ void load(const uint8_t* __restrict__ src, size_t begin, size_t nbytes, size_t limit,
                                         uint32_t lane) {
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i) {
            const size_t off = begin + 1024 * i + 16 * lane;
            const bool ok = 1024 * i + 16 * lane < nbytes && off + 16 <= limit;
            const uint4 x = *(const uint4*)(src + (ok ? off : 0));
            v[i] = ok ? x : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    __device__ __forceinline__ void store(uint8_t* dst, size_t nbytes, uint32_t lane) const {
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i)
            if (1024 * i + 16 * lane < nbytes) *(uint4*)(dst + 1024 * i + 16 * lane) = v[i];
    }
};

// --------------------------------------------------------------------- Q8_0
// One wave's share of the TPW 16-row tiles t0 .. t0+TPW-1 (tile t0 + tt at
// wt + tt*tstride; an index past the last tile reads tile t0 and is not
// stored): chunks gbeg, gbeg+1, ... (GPW per pass, passes gstep apart),
// accumulated into acc[tt] (one value per naccs slot).  Every staged
// activation chunk serves the TPW tiles' weights (TPW = 2 halves the
// activation bytes per weight byte).  xs / as: the wave's LDS slice for
// staged scales and activation bytes.  P = 2: the activation holds 2M layout
// rows (two pieces per token).
template <int MT, int P, bool DOTS, int GPW, int TPW>
__device__ __forceinline__ void q8_0_wave(const uint8_t* __restrict__ wt, size_t tstride,
                                          const uint8_t* __restrict__ act, int32_t* __restrict__ dots, uint32_t t0,
                                          uint32_t M, uint32_t N, uint32_t K, uint32_t nG, uint32_t xd_off,
                                          uint32_t gbeg, uint32_t gstep, uint32_t gend, float* xs, uint8_t* as,
                                          float (&acc)[TPW][4]) {
    constexpr int R = naccs<MT, P>();
    constexpr int S = slots<MT>();
    constexpr int NA = ngroups<MT, P>();
    constexpr int NB = 4 * GPW;
    constexpr int ACT_MAX = GPW * 128 * lrows<MT, P>();  // act bytes per wave pass
    const uint32_t lane = threadIdx.x & 63, row = lane & 15, g = lane >> 4;
    const uint32_t VR = P * M;  // layout rows
    const size_t act_bytes = (size_t)nG * 128 * VR;
    for (uint32_t G0 = gbeg; G0 < gend; G0 += gstep) {
        ScaleStage<NB, S, P == 2> sc;
        ByteStage<ACT_MAX> ast;
        if constexpr (!DOTS) sc.load((const float*)(act + xd_off), nG * 4, 4 * G0, M, lane);
        ast.load(act, (size_t)G0 * 128 * VR, (size_t)GPW * 128 * VR, act_bytes, lane);
        uint4 b01[GPW][TPW], b23[GPW][TPW];
        uint2 dw[GPW][TPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint32_t G = min(G0 + u, gend - 1);
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                const uint8_t* ch = wt + tt * tstride + (size_t)G * kQ8TChunk;
                b01[u][tt] = ld_stream16(ch + lane * 16);
                b23[u][tt] = ld_stream16(ch + 1024 + lane * 16);
                dw[u][tt] = ld_stream8(ch + 2048 + row * 8);
            }
        }
        if constexpr (!DOTS) sc.store(xs, lane);
        ast.store(as, (size_t)GPW * 128 * VR, lane);
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint32_t G = G0 + u;
            if (G >= gend) break;
            long A[NA][4];
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                const uint32_t va = 16 * a + row;
                const bool aval = va < VR;
                const uint8_t* ap = as + (((size_t)u * 4 + g) * VR + (aval ? va : 0)) * 32;
                const uint4 a01 = *(const uint4*)ap;
                const uint4 a23 = *(const uint4*)(ap + 16);
                A[a][0] = aval ? pack2(a01.x, a01.y) : 0l;
                A[a][1] = aval ? pack2(a01.z, a01.w) : 0l;
                A[a][2] = aval ? pack2(a23.x, a23.y) : 0l;
                A[a][3] = aval ? pack2(a23.z, a23.w) : 0l;
            }
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
            const long B[4] = {pack2(b01[u][tt].x, b01[u][tt].y), pack2(b01[u][tt].z, b01[u][tt].w),
                               pack2(b23[u][tt].x, b23[u][tt].y), pack2(b23[u][tt].z, b23[u][tt].w)};
            const float dwf[4] = {h2f(dw[u][tt].x & 0xFFFF), h2f(dw[u][tt].x >> 16), h2f(dw[u][tt].y & 0xFFFF),
                                  h2f(dw[u][tt].y >> 16)};
            float(&ac)[4] = acc[tt];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v4i cc[NA];
#pragma unroll
                for (int a = 0; a < NA; ++a) cc[a] = mfma_i8(A[a][j], B[j]);
                const uint32_t b = 4 * G + j;
                if constexpr (DOTS) {
                    const uint32_t n = 16 * (t0 + tt) + row, nb = K / 32;
                    if (n < N && b < nb)
                        for (int a = 0; a < NA; ++a)
                            for (int r = 0; r < 4; ++r) {
                                const uint32_t vr = 16 * a + 4 * g + r;
                                if (vr < VR) dots[((size_t)vr * N + n) * nb + b] = cc[a][r];
                            }
                } else if constexpr (MT == 1 && P == 1) {
                    ac[0] = fmaf((float)cc[0][0], dwf[j] * xs[4 * u + j], ac[0]);
                } else if constexpr (MT == 1) {  // P = 2: D rows 0, 1 of lanes 0-15
                    ac[0] = fmaf((float)(cc[0][0] * 256 + cc[0][1]), dwf[j] * xs[4 * u + j], ac[0]);
                } else if constexpr (P == 1) {
                    const float4 dx =
                        (4 * g < S) ? *(const float4*)(xs + (4 * u + j) * S + 4 * g) : make_float4(0.f, 0.f, 0.f, 0.f);
                    const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                    for (int r = 0; r < R; ++r) ac[r] = fmaf((float)cc[0][r], dwf[j] * dxv[r], ac[r]);
                } else {
#pragma unroll
                    for (int a = 0; a < NA; ++a) {
                        const uint32_t tk = 8 * a + 2 * g;  // tokens tk, tk + 1 (scales pre-divided by 256)
                        const float2 dx =
                            (tk < (uint32_t)S) ? *(const float2*)(xs + (4 * u + j) * S + tk) : make_float2(0.f, 0.f);
                        ac[2 * a] = fmaf((float)(cc[a][0] * 256 + cc[a][1]), dwf[j] * dx.x, ac[2 * a]);
                        ac[2 * a + 1] = fmaf((float)(cc[a][2] * 256 + cc[a][3]), dwf[j] * dx.y, ac[2 * a + 1]);
                    }
                }
            }
            }
        }
    }
}

// LDS floats of one wave's slice (scales + activation bytes).
template <int MT, int P, int GPW>
constexpr uint32_t q8_wave_lds() { return 4 * GPW * slots<MT>() + GPW * 128 * lrows<MT, P>() / 4; }

// grid = (groups of TPW 16-row tiles, K splits): workgroup (b, sp) covers
// chunks [sp*nG/ns, (sp+1)*nG/ns) of tiles TPW*b .. TPW*b+TPW-1 (ns =
// gridDim.y), split over its nw waves, and writes its sums to y +
// sp*split_stride (one partial result per split; ns = 1: the whole K range).
template <int MT, int P, bool DOTS, int GPW, int TPW>
__global__ __launch_bounds__(1024) void k_mv_q8_0(const uint8_t* __restrict__ W, const uint8_t* __restrict__ act,
                                                  float* __restrict__ y, int32_t* __restrict__ dots, uint32_t M,
                                                  uint32_t N, uint32_t K, uint32_t nG, uint32_t xd_off, uint32_t ldy,
                                                  int accumulate, size_t split_stride) {
    extern __shared__ float lds[];
    constexpr int R = naccs<MT, P>();
    const uint32_t t0 = TPW * blockIdx.x, sp = blockIdx.y;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t g0 = sp * nG / gridDim.y, g1 = (sp + 1) * nG / gridDim.y;
    const uint32_t nT = (N + 15) / 16;
    float* red = lds;
    float* xs = lds + TPW * nw * 256 + w * q8_wave_lds<MT, P, GPW>();
    uint8_t* as = (uint8_t*)(xs + 4 * GPW * slots<MT>());
    float acc[TPW][4] = {};
    // a second tile past the last one reads the first (its rows are not stored)
    const size_t tstride = TPW > 1 && t0 + 1 < nT ? (size_t)nG * kQ8TChunk : 0;
    q8_0_wave<MT, P, DOTS, GPW, TPW>(W + (size_t)t0 * nG * kQ8TChunk, tstride, act, dots, t0, M, N, K, nG, xd_off,
                                     g0 + w * GPW, nw * GPW, g1, xs, as, acc);
    if constexpr (!DOTS) reduce_store<R, P, TPW>(acc, red, y + sp * split_stride, t0, M, N, ldy, accumulate);
}

// Sum of v over lanes l, l^16, l^32, l^48, in every lane: v_permlane32_swap
// pairs lanes 0-31 with 32-63 and v_permlane16_swap odd with even 16-lane
// rows, each returning both halves; every lane adds the same two operands.
__device__ __forceinline__ float sum_lane_groups(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Lane 16*(lane/16) + K's value in every lane of its 16-lane row (DPP
// row_newbcast:K).
template <int K>
__device__ __forceinline__ uint32_t row_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x150 + K, 0xF, 0xF, false);
}

// M = 1, one piece, one K range (the decode matvec of a single sequence):
// every MFMA A row carries the token, so every lane holds its weight row's
// four block dots of a chunk, and lane group g applies the epilogue of block
// g only (one conversion, scale and FMA per chunk instead of four), the four
// groups' partials added once at the end.  The activation operand skips LDS:
// lane 16g + k loads dword k % 8 of group g's 32 bytes in chunk G0 + k/8 (a
// wave's loads cover two chunks with no repeated byte), and lane group g's
// operand for a chunk -- those 8 dwords -- is what its own 16-lane row loaded,
// taken with row broadcasts.  Loads: activation and scales first, weights
// after, all before any compute (a clamped index past the range reads the
// last chunk again and enters with a zero scale).
template <int GPW>
__global__ __launch_bounds__(1024) void k_mv_q8_0_m1(const uint8_t* __restrict__ W, const uint8_t* __restrict__ act,
                                                     float* __restrict__ y, uint32_t N, uint32_t nG, uint32_t xd_off,
                                                     int accumulate) {
    extern __shared__ float lds[];  // [nw][16] wave partials
    constexpr int NPAIR = (GPW + 1) / 2;
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63, row = lane & 15, g = lane >> 4;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint8_t* wt = W + (size_t)t * nG * kQ8TChunk;
    const float* xd = (const float*)(act + xd_off);  // token 0's block scales
    const uint32_t* a32 = (const uint32_t*)act;
    float acc = 0.0f;
    for (uint32_t G0 = w * GPW; G0 < nG; G0 += nw * GPW) {
        uint32_t av[NPAIR];
        float dxg[GPW];
#pragma unroll
        for (int pr = 0; pr < NPAIR; ++pr) {
            const uint32_t G = min(G0 + 2 * pr + (row >> 3), nG - 1);
            av[pr] = a32[(4 * G + g) * 8 + (row & 7)];
        }
#pragma unroll
        for (int u = 0; u < GPW; ++u) dxg[u] = xd[4 * min(G0 + u, nG - 1) + g];
        __builtin_amdgcn_sched_barrier(0);  // activation loads complete first (in-order returns)
        uint4 b01[GPW], b23[GPW];
        uint2 dw[GPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint8_t* ch = wt + (size_t)min(G0 + u, nG - 1) * kQ8TChunk;
            b01[u] = ld_stream16(ch + lane * 16);
            b23[u] = ld_stream16(ch + 1024 + lane * 16);
            dw[u] = ld_stream8(ch + 2048 + row * 8);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the pass before any compute
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint32_t v = av[u / 2];
            uint32_t aw[8];  // the chunk's 8 dwords: lanes 8 (u % 2) .. +7 of the row
#define EC_BC(i) aw[i] = (u & 1) ? row_bcast<8 + i>(v) : row_bcast<i>(v);
            EC_BC(0) EC_BC(1) EC_BC(2) EC_BC(3) EC_BC(4) EC_BC(5) EC_BC(6) EC_BC(7)
#undef EC_BC
            const long B[4] = {pack2(b01[u].x, b01[u].y), pack2(b01[u].z, b01[u].w), pack2(b23[u].x, b23[u].y),
                               pack2(b23[u].z, b23[u].w)};
            int dot[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dot[j] = mfma_i8(pack2(aw[2 * j], aw[2 * j + 1]), B[j])[0];
            const int dg = g == 0 ? dot[0] : g == 1 ? dot[1] : g == 2 ? dot[2] : dot[3];
            // block g's fp16 scale, by masks (a select on g becomes a stack-indexed load)
            const uint32_t hm = (g & 2) ? 0xFFFFFFFFu : 0u;
            const uint32_t h = dw[u].x ^ ((dw[u].x ^ dw[u].y) & hm);
            const float dwf = h2f((uint16_t)(h >> (16 * (g & 1))));
            const float dx = G0 + u < nG ? dxg[u] : 0.0f;
            acc = fmaf((float)dg, dwf * dx, acc);
        }
    }
    acc = sum_lane_groups(acc);
    const uint32_t n = 16 * t + row;
    if (nw == 1) {
        if (lane < 16 && n < N) y[n] = accumulate ? y[n] + acc : acc;
        return;
    }
    if (lane < 16) lds[w * 16 + lane] = acc;
    __syncthreads();
    if (threadIdx.x < 16 && 16 * t + threadIdx.x < N) {
        const uint32_t nn = 16 * t + threadIdx.x;
        float sm = lds[threadIdx.x];
        for (uint32_t v = 1; v < nw; ++v) sm += lds[v * 16 + threadIdx.x];
        y[nn] = accumulate ? y[nn] + sm : sm;
    }
}

// --------------------------------------------------------------------- Q4_K
// The eight 6-bit (scale, min) pairs of a super-block from its 12 scale bytes
// (q[0] = bytes 0-3, ...), four per dword: sc[0] holds sub-blocks 0-3 (byte s
// = scale of sub-block s), sc[1] sub-blocks 4-7, mn likewise -- the unpack of
// src/kernels/quant.cpp:222-242 done on four bytes per operation.
__device__ __forceinline__ void q4k_scale_min4(const uint32_t (&q)[3], uint32_t (&sc)[2], uint32_t (&mn)[2]) {
    sc[0] = q[0] & 0x3F3F3F3Fu;
    mn[0] = q[1] & 0x3F3F3F3Fu;
    sc[1] = (q[2] & 0x0F0F0F0Fu) | ((q[0] >> 2) & 0x30303030u);
    mn[1] = ((q[2] >> 4) & 0x0F0F0F0Fu) | ((q[1] >> 2) & 0x30303030u);
}

__device__ __forceinline__ void q4k_scale_min(const uint32_t (&q)[3], int s, uint32_t& sc, uint32_t& m) {
    // q holds scales[0..11] little-endian: byte i = (q[i/4] >> 8*(i%4)) & 0xFF
    auto byte = [&](int i) -> uint32_t { return (q[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
    if (s < 4) {
        sc = byte(s) & 63u;
        m = byte(s + 4) & 63u;
    } else {
        sc = (byte(s + 4) & 0x0Fu) | ((byte(s - 4) >> 6) << 4);
        m = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
    }
}


// M = 1 (the epilogue split, !DOTS): one token leaves 15 of the MFMA's 16 A
// rows free, so every A row carries the token (row r: layout row r % P, i.e.
// piece r % 2 for P = 2) and every lane holds its weight row's sub-block dots;
// lane group g (lanes 16g .. 16g+15) applies the epilogue of sub-blocks g and
// 4+g only -- a quarter of the per-sub-block instructions -- and the four
// groups' fp32 partials are added once at the end.
// TPW 16-row tiles per wave (MT > 1, !DOTS): each staged activation
// super-block serves the TPW tiles' weights (tile t0 + tt at wt + tt *
// tstride; a second tile past the last one reads the first and is not
// stored).
template <int MT, int P, bool DOTS, int GPW, int TPW>
__global__ __launch_bounds__(1024) void k_mv_q4_K(const uint8_t* __restrict__ W, const uint8_t* __restrict__ act,
                                                  float* __restrict__ y, int32_t* __restrict__ dots, uint32_t M,
                                                  uint32_t N, uint32_t K, uint32_t nB, uint32_t xd_off,
                                                  uint32_t dxs_off, uint32_t ldy, int accumulate) {
    extern __shared__ float lds[];
    constexpr int R = naccs<MT, P>();
    constexpr int S = slots<MT>();
    constexpr int NA = ngroups<MT, P>();
    constexpr int NB = 8 * GPW;
    static_assert(TPW == 1 || (MT > 1 && !DOTS), "two tiles per wave: M > 1, no dots output");
    const uint32_t t = TPW * blockIdx.x, lane = threadIdx.x & 63, row = lane & 15, g = lane >> 4;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = blockDim.x >> 6;
    constexpr int ACT_MAX = GPW * 256 * lrows<MT, P>();
    float* red = lds;
    float* xs = lds + TPW * nw * 256 + w * (2 * NB * S + ACT_MAX / 4);
    float* xms = xs + NB * S;
    uint8_t* as = (uint8_t*)(xms + NB * S);
    const uint8_t* wt = W + (size_t)t * nB * kQ4TChunk;
    const uint32_t nT = (N + 15) / 16;
    const size_t tstride = TPW > 1 && t + 1 < nT ? (size_t)nB * kQ4TChunk : 0;
    const uint32_t VR = P * M;  // layout rows
    const size_t act_bytes = (size_t)nB * 256 * VR;
    float acc4[TPW][4] = {};
    float(&acc)[4] = acc4[0];

    for (uint32_t B0 = w * GPW; B0 < nB; B0 += nw * GPW) {
        ScaleStage<NB, S, P == 2> sd;
        ScaleStage<NB, S> sm;
        ByteStage<ACT_MAX> ast;
        if constexpr (!DOTS) {
            sd.load((const float*)(act + xd_off), nB * 8, 8 * B0, M, lane);
            sm.load((const float*)(act + dxs_off), nB * 8, 8 * B0, M, lane);
        }
        ast.load(act, (size_t)B0 * 256 * VR, (size_t)GPW * 256 * VR, act_bytes, lane);
        uint4 q0[GPW][TPW], q1[GPW][TPW], hdr[GPW][TPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint32_t b = min(B0 + u, nB - 1);
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                const uint8_t* ch = wt + tt * tstride + (size_t)b * kQ4TChunk;
                q0[u][tt] = ld_stream16(ch + lane * 16);
                q1[u][tt] = ld_stream16(ch + 1024 + lane * 16);
                hdr[u][tt] = ld_stream16(ch + 2048 + row * 16);
            }
        }
        if constexpr (!DOTS) {
            sd.store(xs, lane);
            sm.store(xms, lane);
        }
        ast.store(as, (size_t)GPW * 256 * VR, lane);
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint32_t b = B0 + u;
            if (b >= nB) break;
            uint32_t aw[NA][16];
            bool aval[NA];
            constexpr bool SPLIT = MT == 1 && !DOTS;
#pragma unroll
            for (int ga = 0; ga < NA; ++ga) {
                const uint32_t va = SPLIT ? row % P : 16 * ga + row;
                aval[ga] = SPLIT || va < VR;
                const uint8_t* ap = as + (((size_t)u * 4 + g) * VR + (aval[ga] ? va : 0)) * 64;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 a4 = *(const uint4*)(ap + 16 * i);
                    aw[ga][4 * i] = a4.x, aw[ga][4 * i + 1] = a4.y, aw[ga][4 * i + 2] = a4.z, aw[ga][4 * i + 3] = a4.w;
                }
            }
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
            float(&acc)[4] = acc4[tt];
            const uint32_t qw[8] = {q0[u][tt].x, q0[u][tt].y, q0[u][tt].z, q0[u][tt].w,
                                    q1[u][tt].x, q1[u][tt].y, q1[u][tt].z, q1[u][tt].w};
            const float d = h2f(hdr[u][tt].x & 0xFFFF), dmin = h2f(hdr[u][tt].x >> 16);
            const uint32_t scb[3] = {hdr[u][tt].y, hdr[u][tt].z, hdr[u][tt].w};
            uint32_t sc4[2], mn4[2];
            q4k_scale_min4(scb, sc4, mn4);
            float a_sc = 0.0f, a_mn = 0.0f;  // M = 1: sum_s sc_s*dot_s*dx_s and sum_s m_s*dxs_s, scaled once
            int dsplit[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint32_t lo = qw[s] & 0x0F0F0F0Fu, hi = (qw[s] >> 4) & 0x0F0F0F0Fu;
                v4i cc[NA];
#pragma unroll
                for (int ga = 0; ga < NA; ++ga)
                    cc[ga] = mfma_i8(aval[ga] ? pack2(aw[ga][2 * s], aw[ga][2 * s + 1]) : 0l, pack2(lo, hi));
                const uint32_t sbi = 8 * b + s;
                if constexpr (DOTS) {
                    const uint32_t n = 16 * t + row, nsb = K / 32;
                    if (n < N && sbi < nsb)
                        for (int ga = 0; ga < NA; ++ga)
                            for (int r = 0; r < 4; ++r) {
                                const uint32_t vr = 16 * ga + 4 * g + r;
                                if (vr < VR) dots[((size_t)vr * N + n) * nsb + sbi] = cc[ga][r];
                            }
                } else {
                    const uint32_t scv = (sc4[s >> 2] >> (8 * (s & 3))) & 0xFFu;
                    const uint32_t mnv = (mn4[s >> 2] >> (8 * (s & 3))) & 0xFFu;
                    const int e = 8 * u + s;
                    if constexpr (MT == 1) {
                        dsplit[s] = P == 2 ? cc[0][0] * 256 + cc[0][1] : cc[0][0];  // |dot| <= 2^19 per piece
                    } else if constexpr (P == 2) {
                        const float dsc = d * (float)scv, dmn = dmin * (float)mnv;
#pragma unroll
                        for (int ga = 0; ga < NA; ++ga) {
                            const uint32_t t0 = 8 * ga + 2 * g;  // tokens t0, t0 + 1
                            const bool ok = t0 < (uint32_t)S;
                            const float2 dx = ok ? *(const float2*)(xs + e * S + t0) : make_float2(0.f, 0.f);
                            const float2 dm = ok ? *(const float2*)(xms + e * S + t0) : make_float2(0.f, 0.f);
                            acc[2 * ga] = fmaf((float)(cc[ga][0] * 256 + cc[ga][1]), dsc * dx.x, acc[2 * ga]);
                            acc[2 * ga] = fmaf(-dmn, dm.x, acc[2 * ga]);
                            acc[2 * ga + 1] = fmaf((float)(cc[ga][2] * 256 + cc[ga][3]), dsc * dx.y, acc[2 * ga + 1]);
                            acc[2 * ga + 1] = fmaf(-dmn, dm.y, acc[2 * ga + 1]);
                        }
                    } else {
                        const float dsc = d * (float)scv, dmn = dmin * (float)mnv;
                        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
                        const float4 dx = (4 * g < S) ? *(const float4*)(xs + e * S + 4 * g) : z4;
                        const float4 dm = (4 * g < S) ? *(const float4*)(xms + e * S + 4 * g) : z4;
                        const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
                        const float dmv[4] = {dm.x, dm.y, dm.z, dm.w};
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            acc[r] = fmaf((float)cc[0][r], dsc * dxv[r], acc[r]);
                            acc[r] = fmaf(-dmn, dmv[r], acc[r]);
                        }
                    }
                }
            }
            if constexpr (MT == 1 && !DOTS) {
                // lane group g: sub-blocks g and 4 + g
                const int da = g == 0 ? dsplit[0] : g == 1 ? dsplit[1] : g == 2 ? dsplit[2] : dsplit[3];
                const int db = g == 0 ? dsplit[4] : g == 1 ? dsplit[5] : g == 2 ? dsplit[6] : dsplit[7];
                const uint32_t sh = 8 * g;
                const int ea = 8 * u + g, eb = ea + 4;
                a_sc = (float)da * ((float)((sc4[0] >> sh) & 0xFFu) * xs[ea]);
                a_sc = fmaf((float)db, (float)((sc4[1] >> sh) & 0xFFu) * xs[eb], a_sc);
                a_mn = (float)((mn4[0] >> sh) & 0xFFu) * xms[ea];
                a_mn = fmaf((float)((mn4[1] >> sh) & 0xFFu), xms[eb], a_mn);
                acc[0] = fmaf(d, a_sc, acc[0]);
                acc[0] = fmaf(-dmin, a_mn, acc[0]);
            }
            }
        }
    }
    if constexpr (MT == 1 && !DOTS) acc[0] = sum_lane_groups(acc[0]);
    if constexpr (!DOTS) reduce_store<R, P, TPW>(acc4, red, y, t, M, N, ldy, accumulate);
}


// M = 1, one activation piece, without LDS staging: the k_mv_q4_K<1, 1>
// arithmetic (every MFMA A row carries the token, lane group g applies the
// epilogue of sub-blocks g and 4+g, the groups' partials added at the end)
// with the activation operand fetched once per wave: lane l loads dword l of
// the super-block's 256 activation bytes (one coalesced 256-byte load), and
// lane group g, whose A operand is dwords 16g .. 16g+15 -- exactly the
// dwords its own 16-lane row loaded -- takes them with 16 row broadcasts.
// The group's two sub-block scales and d_x*sum values are loaded per lane.
// Loads are issued activation first, weights after, all before any compute
// (no branch: a clamped index past the range reads the last super-block and
// enters with d = dmin = 0).
template <int GPW>
__global__ __launch_bounds__(1024) void k_mv_q4_K_m1(const uint8_t* __restrict__ W, const uint8_t* __restrict__ act,
                                                     float* __restrict__ y, uint32_t N, uint32_t nB, uint32_t xd_off,
                                                     uint32_t dxs_off, int accumulate) {
    extern __shared__ float lds[];  // [nw][16] wave partials
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63, row = lane & 15, g = lane >> 4;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint8_t* wt = W + (size_t)t * nB * kQ4TChunk;
    const float* xd = (const float*)(act + xd_off);   // token 0's sub-block scales
    const float* xm = (const float*)(act + dxs_off);  // token 0's d_x * sum(q) per sub-block
    float acc = 0.0f;
    for (uint32_t B0 = w * GPW; B0 < nB; B0 += nw * GPW) {
        uint32_t bb[GPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) bb[u] = min(B0 + u, nB - 1);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t av[GPW];
        float dxa[GPW], dxb[GPW], dma[GPW], dmb[GPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            av[u] = ((const uint32_t*)(act + (size_t)bb[u] * 256))[lane];
            dxa[u] = xd[8 * bb[u] + g], dxb[u] = xd[8 * bb[u] + 4 + g];
            dma[u] = xm[8 * bb[u] + g], dmb[u] = xm[8 * bb[u] + 4 + g];
        }
        __builtin_amdgcn_sched_barrier(0);  // activation loads complete first (in-order returns)
        uint4 q0[GPW], q1[GPW], hdr[GPW];
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const uint8_t* ch = wt + (size_t)bb[u] * kQ4TChunk;
            q0[u] = ld_stream16(ch + lane * 16);
            q1[u] = ld_stream16(ch + 1024 + lane * 16);
            hdr[u] = ld_stream16(ch + 2048 + row * 16);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the pass before any compute
#pragma unroll
        for (int u = 0; u < GPW; ++u) {
            const bool live = B0 + u < nB;
            const uint32_t aw[16] = {row_bcast<0>(av[u]),  row_bcast<1>(av[u]),  row_bcast<2>(av[u]),
                                     row_bcast<3>(av[u]),  row_bcast<4>(av[u]),  row_bcast<5>(av[u]),
                                     row_bcast<6>(av[u]),  row_bcast<7>(av[u]),  row_bcast<8>(av[u]),
                                     row_bcast<9>(av[u]),  row_bcast<10>(av[u]), row_bcast<11>(av[u]),
                                     row_bcast<12>(av[u]), row_bcast<13>(av[u]), row_bcast<14>(av[u]),
                                     row_bcast<15>(av[u])};
            const uint32_t qw[8] = {q0[u].x, q0[u].y, q0[u].z, q0[u].w, q1[u].x, q1[u].y, q1[u].z, q1[u].w};
            int dot[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint32_t lo = qw[s] & 0x0F0F0F0Fu, hi = (qw[s] >> 4) & 0x0F0F0F0Fu;
                dot[s] = mfma_i8(pack2(aw[2 * s], aw[2 * s + 1]), pack2(lo, hi))[0];
            }
            const int da = g == 0 ? dot[0] : g == 1 ? dot[1] : g == 2 ? dot[2] : dot[3];
            const int db = g == 0 ? dot[4] : g == 1 ? dot[5] : g == 2 ? dot[6] : dot[7];
            const uint32_t scb[3] = {hdr[u].y, hdr[u].z, hdr[u].w};
            uint32_t sc4[2], mn4[2];
            q4k_scale_min4(scb, sc4, mn4);
            const uint32_t sh = 8 * g;
            float a_sc = (float)da * ((float)((sc4[0] >> sh) & 0xFFu) * dxa[u]);
            a_sc = fmaf((float)db, (float)((sc4[1] >> sh) & 0xFFu) * dxb[u], a_sc);
            float a_mn = (float)((mn4[0] >> sh) & 0xFFu) * dma[u];
            a_mn = fmaf((float)((mn4[1] >> sh) & 0xFFu), dmb[u], a_mn);
            const float d = live ? h2f(hdr[u].x & 0xFFFF) : 0.0f, dmin = live ? h2f(hdr[u].x >> 16) : 0.0f;
            acc = fmaf(d, a_sc, acc);
            acc = fmaf(-dmin, a_mn, acc);
        }
    }
    acc = sum_lane_groups(acc);
    const uint32_t n = 16 * t + row;
    if (nw == 1) {
        if (lane < 16 && n < N) y[n] = accumulate ? y[n] + acc : acc;
        return;
    }
    if (lane < 16) lds[w * 16 + lane] = acc;
    __syncthreads();
    if (threadIdx.x < 16 && 16 * t + threadIdx.x < N) {
        const uint32_t nn = 16 * t + threadIdx.x;
        float s = lds[threadIdx.x];
        for (uint32_t v = 1; v < nw; ++v) s += lds[v * 16 + threadIdx.x];
        y[nn] = accumulate ? y[nn] + s : s;
    }
}

// ------------------------------------------------ reference-semantics fp32 path
int gguf_mv_fast(int fmt, const uint8_t* W, const float* x, float* y, uint32_t M, uint32_t K, hipStream_t st);

// One wave per output row, fp32 activations, GGUF bytes read in place.
// Q8_0 follows src/kernels/matvec.cpp:62-87 per block; Q4_K :92-142; Q2_K
// :146-183; F16 :18-45.  The row sum is a wave reduction (order differs from
// the reference's sequential loop by rounding only).
__device__ __forceinline__ uint16_t ld16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

__global__ __launch_bounds__(64) void k_matvec_gguf_f32(int fmt, const uint8_t* __restrict__ Wb,
                                                        const float* __restrict__ x, float* __restrict__ y,
                                                        uint32_t M, uint32_t K) {
    const uint32_t m = blockIdx.x, lane = threadIdx.x;
    if (m >= M) return;
    float sum = 0.0f;
    if (fmt == EC_Q8_0) {
        const uint32_t nb = K / 32;
        const uint8_t* row = Wb + (size_t)m * nb * 34;
        for (uint32_t b = lane; b < nb; b += 64) {
            const uint8_t* bp = row + (size_t)b * 34;
            const float d = h2f(ld16(bp));
            float bs = 0.0f;
            for (int j = 0; j < 32; ++j) bs = fmaf((float)(int8_t)bp[2 + j], x[32 * b + j], bs);
            sum = fmaf(d, bs, sum);
        }
    } else if (fmt == EC_Q4_K) {
        const uint32_t nb = K / 256;
        const uint8_t* row = Wb + (size_t)m * nb * 144;
        for (uint32_t b = lane; b < nb * 4; b += 64) {  // one 64-weight group per lane step
            const uint32_t sbk = b / 4, blk = b % 4;
            const uint8_t* bp = row + (size_t)sbk * 144;
            const float d = h2f(ld16(bp)), dmin = h2f(ld16(bp + 2));
            const uint32_t scw[3] = {(uint32_t)bp[4] | (uint32_t)bp[5] << 8 | (uint32_t)bp[6] << 16 | (uint32_t)bp[7] << 24,
                                     (uint32_t)bp[8] | (uint32_t)bp[9] << 8 | (uint32_t)bp[10] << 16 | (uint32_t)bp[11] << 24,
                                     (uint32_t)bp[12] | (uint32_t)bp[13] << 8 | (uint32_t)bp[14] << 16 | (uint32_t)bp[15] << 24};
            uint32_t sc0, mn0, sc1, mn1;
            q4k_scale_min(scw, 2 * blk, sc0, mn0);
            q4k_scale_min(scw, 2 * blk + 1, sc1, mn1);
            const float rs0 = d * (float)sc0, rm0 = dmin * (float)mn0, rs1 = d * (float)sc1, rm1 = dmin * (float)mn1;
            const uint8_t* qs = bp + 16 + 32 * blk;
            const float* xb = x + 256 * sbk + 64 * blk;
            for (int j = 0; j < 16; ++j) {
                sum = fmaf(rs0 * (float)(qs[j] & 0x0F) - rm0, xb[j], sum);
                sum = fmaf(rs1 * (float)(qs[16 + j] & 0x0F) - rm1, xb[16 + j], sum);
                sum = fmaf(rs0 * (float)(qs[j] >> 4) - rm0, xb[32 + j], sum);
                sum = fmaf(rs1 * (float)(qs[16 + j] >> 4) - rm1, xb[48 + j], sum);
            }
        }
    } else if (fmt == EC_Q2_K) {
        const uint32_t nb = K / 256;
        const uint8_t* row = Wb + (size_t)m * nb * 84;
        for (uint32_t b = lane; b < nb * 32; b += 64) {  // one 8-weight sub-block per lane step
            const uint32_t sbk = b / 32, sb = b % 32;
            const uint8_t* bp = row + (size_t)sbk * 84;
            const float d_all = h2f(ld16(bp)), m_all = h2f(ld16(bp + 2));
            const uint8_t* sc = bp + 4;
            const uint8_t* qs = bp + 20;
            const uint32_t s = sb / 2;
            const uint8_t sv = (sb % 2 == 0) ? sc[s] : sc[s + 8];
            const float scale = d_all * (float)(sv & 0x0F), minv = m_all * (float)(sv >> 4);
            for (int i = 0; i < 8; ++i) {
                const uint32_t j = 8 * sb + i;
                const int q = (qs[j / 4] >> ((j % 4) * 2)) & 3;
                sum = fmaf(scale * (float)q - minv, x[256 * sbk + j], sum);
            }
        }
    } else {  // F16 rows
        const uint16_t* row = (const uint16_t*)Wb + (size_t)m * K;
        for (uint32_t k = lane; k < K; k += 64) sum = fmaf(h2f(row[k]), x[k], sum);
    }
    sum = wave_sum(sum);
    if (lane == 0) y[m] += sum;
}

// scores[p] = sum_k K[p][k] * scale[p] * q[k]  (src/kernels/quant.cpp:100-144)
__global__ void k_dequant_dot_int8(const float* __restrict__ q, const int8_t* __restrict__ keys,
                                   const float* __restrict__ scales, float* __restrict__ scores, uint32_t dim,
                                   uint32_t seq) {
    const uint32_t p = blockIdx.x, lane = threadIdx.x;
    if (p >= seq) return;
    const int8_t* kp = keys + (size_t)p * dim;
    const float s = scales[p];
    float acc = 0.0f;
    for (uint32_t k = lane; k < dim; k += 64) acc = fmaf((float)kp[k] * s, q[k], acc);
    acc = wave_sum(acc);
    if (lane == 0) scores[p] = acc;
}

// GGUF blocks -> fp16, one thread per block (src/kernels/quant.cpp:308-396).
__global__ void k_dequant_fp16(int fmt, const uint8_t* __restrict__ src, uint16_t* __restrict__ dst, size_t nblk) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    if (fmt == EC_Q8_0) {
        const uint8_t* bp = src + b * 34;
        const float d = h2f(ld16(bp));
        for (int j = 0; j < 32; ++j) dst[b * 32 + j] = __half_as_ushort(__float2half_rn(d * (float)(int8_t)bp[2 + j]));
    } else if (fmt == EC_Q4_K) {
        const uint8_t* bp = src + b * 144;
        const float d = h2f(ld16(bp)), dmin = h2f(ld16(bp + 2));
        uint32_t scw[3];
        for (int i = 0; i < 3; ++i)
            scw[i] = (uint32_t)bp[4 + 4 * i] | (uint32_t)bp[5 + 4 * i] << 8 | (uint32_t)bp[6 + 4 * i] << 16 |
                     (uint32_t)bp[7 + 4 * i] << 24;
        for (int blk = 0; blk < 4; ++blk) {
            uint32_t sc0, mn0, sc1, mn1;
            q4k_scale_min(scw, 2 * blk, sc0, mn0);
            q4k_scale_min(scw, 2 * blk + 1, sc1, mn1);
            const float rs0 = d * (float)sc0, rm0 = dmin * (float)mn0, rs1 = d * (float)sc1, rm1 = dmin * (float)mn1;
            const uint8_t* qs = bp + 16 + 32 * blk;
            uint16_t* o = dst + b * 256 + 64 * blk;
            for (int j = 0; j < 16; ++j) {
                o[j] = __half_as_ushort(__float2half_rn(rs0 * (float)(qs[j] & 0x0F) - rm0));
                o[16 + j] = __half_as_ushort(__float2half_rn(rs1 * (float)(qs[16 + j] & 0x0F) - rm1));
                o[32 + j] = __half_as_ushort(__float2half_rn(rs0 * (float)(qs[j] >> 4) - rm0));
                o[48 + j] = __half_as_ushort(__float2half_rn(rs1 * (float)(qs[16 + j] >> 4) - rm1));
            }
        }
    } else {  // Q2_K
        const uint8_t* bp = src + b * 84;
        const float d_all = h2f(ld16(bp)), m_all = h2f(ld16(bp + 2));
        for (int j = 0; j < 256; ++j) {
            const int sb = j / 8, s = sb / 2;
            const uint8_t sv = (sb % 2 == 0) ? bp[4 + s] : bp[4 + s + 8];
            const int q = (bp[20 + j / 4] >> ((j % 4) * 2)) & 3;
            dst[b * 256 + j] =
                __half_as_ushort(__float2half_rn(d_all * (float)(sv & 0x0F) * (float)q - m_all * (float)(sv >> 4)));
        }
    }
}

// Chunks per wave (GPW, compile-time) and waves per 16-row tile (nw <= 16):
// aim for a total wave count with every tile's K range covered by one pass
// where possible.  Q8_0: 12288 waves (EC_MV_TARGET_WAVES overrides; with the
// decode step's split-K projections 12288 measured best of 2048 .. 32768:
// 1.92 ms/step at 2048, 1.86 at 4096, 1.80 at 12288, 1.86 at 24576); Q4_K:
// 3072 (EC_MV_TARGET_WAVES_Q4 overrides; M = 1, us at 1536 / 2048 / 3072 /
// 4096 / 6144: 9216 x 2560 4.83 / 4.83 / 4.76 / 4.75 / 5.14, 12352 x 2560
// 5.52 / 5.51 / 5.51 / 5.93 / 5.94, 2560 x 9216 and 2560 x 4096 flat).
static uint32_t target_waves_q8() {
    static uint32_t v = [] {
        const char* e = getenv("EC_MV_TARGET_WAVES");
        return e ? (uint32_t)atoi(e) : 12288u;
    }();
    return v;
}
// 16-row tiles per wave of the Q8_0 matvec (1, 2 or 4): with one activation
// piece 1 (EC_MV_TPW_P1 overrides), with two 2 (EC_MV_TPW overrides).
static uint32_t tpw_q8(int pieces) {
    static uint32_t v[2] = {[] {
                                const char* e = getenv("EC_MV_TPW_P1");
                                const int t = e ? atoi(e) : 1;
                                return t == 2 || t == 4 ? (uint32_t)t : 1u;
                            }(),
                            [] {
                                const char* e = getenv("EC_MV_TPW");
                                const int t = e ? atoi(e) : 2;
                                return t == 1 || t == 4 ? (uint32_t)t : 2u;
                            }()};
    return v[pieces == 2];
}
// Two tiles per wave with the one-tile plan's chunks per pass (EC_MV_TPW_GPW=full;
// default: half of them, so a wave streams the one-tile plan's weight bytes).
static bool tpw_full_gpw() {
    static bool v = [] {
        const char* e = getenv("EC_MV_TPW_GPW");
        return e && strcmp(e, "full") == 0;
    }();
    return v;
}
static uint32_t tpw_q4() {
    static uint32_t v = [] {
        const char* e = getenv("EC_MV_TPW_Q4");
        return e && atoi(e) == 1 ? 1u : 2u;
    }();
    return v;
}
static uint32_t target_waves_q4() {
    static uint32_t v = [] {
        const char* e = getenv("EC_MV_TARGET_WAVES_Q4");
        return e ? (uint32_t)atoi(e) : 3072u;
    }();
    return v;
}

static void plan(uint32_t n_tiles, uint32_t n_chunks, int max_gpw, int& gpw, uint32_t& nw, uint32_t target) {
    const uint32_t want = (target + n_tiles - 1) / n_tiles;  // waves per tile wanted
    gpw = (int)((n_chunks + want - 1) / (want ? want : 1));
    // one pass per wave where 16 waves can cover the tile's K: a second pass
    // would issue its loads only after the first pass's compute
    const int one_pass = (int)((n_chunks + 15) / 16);
    if (gpw < one_pass) gpw = one_pass;
    if (gpw < 1) gpw = 1;
    if (gpw > max_gpw) gpw = max_gpw;
    nw = (n_chunks + gpw - 1) / gpw;
    if (nw > 16) nw = 16;  // larger K: several passes per wave
}

// LDS per workgroup is 160 KB on gfx950: cap the waves of a workgroup so that
// nw * (reduction slice + wave slice) fits (more passes per wave instead).
constexpr size_t kLdsBytes = 160 * 1024;
static uint32_t lds_cap_waves(uint32_t wave_floats, uint32_t tpw = 1) {
    return (uint32_t)(kLdsBytes / ((256 * tpw + wave_floats) * 4));
}

template <int MT, int P, bool DOTS, int GPW, int TPW>
static void launch_q8_g(const void* W, const void* act, float* y, int32_t* dots, uint32_t M, uint32_t N, uint32_t K,
                        uint32_t ldy, int accumulate, uint32_t nw, uint32_t nsplit, hipStream_t st) {
    const ActLayout L = act_layout(EC_Q8_0, P * M, K);
    const uint32_t nT = round_up(N, 16) / 16, nG = L.Kp / 128;
    nw = min(nw, lds_cap_waves(q8_wave_lds<MT, P, GPW>(), TPW));
    const size_t lds = ((size_t)TPW * nw * 256 + (size_t)nw * q8_wave_lds<MT, P, GPW>()) * sizeof(float);
    hipLaunchKernelGGL((k_mv_q8_0<MT, P, DOTS, GPW, TPW>), dim3((nT + TPW - 1) / TPW, nsplit), dim3(64 * nw), lds, st,
                       (const uint8_t*)W, (const uint8_t*)act, y, dots, M, N, K, nG, (uint32_t)L.xd_off, ldy,
                       accumulate, (size_t)M * ldy);
}

// nsplit > 1 (<= the 128-element chunks of K): the K range is cut into
// nsplit balanced chunk ranges, one workgroup per (tile, range), partial sums
// to y + sp*M*ldy.
// M = 1 with one piece and one K range: k_mv_q8_0_m1 (EC_MV_Q8_M1=staged
// selects k_mv_q8_0, for comparison).
static bool q8_m1_direct() {
    static bool v = [] {
        const char* e = getenv("EC_MV_Q8_M1");
        return !(e && strcmp(e, "staged") == 0);
    }();
    return v;
}

template <int MT, int P, bool DOTS>
static void launch_q8(const void* W, const void* act, float* y, int32_t* dots, uint32_t M, uint32_t N, uint32_t K,
                      uint32_t ldy, int accumulate, hipStream_t st, uint32_t nsplit = 1) {
    const uint32_t nT = round_up(N, 16) / 16, nG = round_up(K, 128) / 128;
    const uint32_t cps = (nG + nsplit - 1) / nsplit;  // longest range
    int gpw;
    uint32_t nw;
    // several tiles per wave: each staged activation chunk serves 16*tpw weight rows (with two pieces
    // the activation bytes of one tile equal its weight bytes), with 1/tpw of the chunks per pass, so a
    // wave streams about the same weight bytes per pass.  GPW <= 5 (two pieces: 4, and 3 for 16 tokens;
    // two tiles: 2): every variant under 128 VGPRs, no spills (two tiles with 3 chunks per pass: lm_head
    // 151936 x 2560, M = 8, 70.2 -> 73.8 us)
    // two tiles per wave only while that leaves >= 128 workgroups: an
    // unsplit 2560 x 9216 at M = 8 (80 two-tile workgroups) runs 12.3 us,
    // with one tile per wave 9.7 us; the decode step's split projections
    // (>= 240 workgroups) keep two
    uint32_t tpw = tpw_q8(P);
    if (tpw > 1 && (nT + tpw - 1) / tpw * nsplit < 128) tpw = 1;
    constexpr int max_gpw = P == 1 || MT == 1 ? 5 : (MT == 16 ? 3 : 4);
    plan(nT * nsplit, cps, max_gpw, gpw, nw, target_waves_q8());
    if constexpr (MT == 1 && P == 1 && !DOTS) {
        if (nsplit == 1 && q8_m1_direct()) {
            const ActLayout L = act_layout(EC_Q8_0, 1, K);
            const size_t lds = (size_t)nw * 16 * sizeof(float);
            switch (gpw) {
#define EC_Q8M1(G)                                                                                            \
    hipLaunchKernelGGL((k_mv_q8_0_m1<G>), dim3(nT), dim3(64 * nw), lds, st, (const uint8_t*)W, (const uint8_t*)act, \
                       y, N, nG, (uint32_t)L.xd_off, accumulate);                                          \
    break;
                case 1: EC_Q8M1(1)
                case 2: EC_Q8M1(2)
                case 3: EC_Q8M1(3)
                case 4: EC_Q8M1(4)
                default: EC_Q8M1(5)
#undef EC_Q8M1
            }
            return;
        }
    }
    if (tpw == 2) {
        const int g2 = min(tpw_full_gpw() ? gpw : (gpw + 1) / 2, 2);
        const uint32_t nw2 = min((cps + g2 - 1) / g2, 16u);
        switch (g2) {
            case 1: launch_q8_g<MT, P, DOTS, 1, 2>(W, act, y, dots, M, N, K, ldy, accumulate, nw2, nsplit, st); break;
            default: launch_q8_g<MT, P, DOTS, 2, 2>(W, act, y, dots, M, N, K, ldy, accumulate, nw2, nsplit, st); break;
        }
        return;
    }
    if (tpw == 4) {
        const uint32_t nw4 = min(cps, 16u);
        launch_q8_g<MT, P, DOTS, 1, 4>(W, act, y, dots, M, N, K, ldy, accumulate, nw4, nsplit, st);
        return;
    }
    switch (gpw) {
        case 1: launch_q8_g<MT, P, DOTS, 1, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, nsplit, st); break;
        case 2: launch_q8_g<MT, P, DOTS, 2, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, nsplit, st); break;
        case 3: launch_q8_g<MT, P, DOTS, 3, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, nsplit, st); break;
        case 4: launch_q8_g<MT, P, DOTS, 4, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, nsplit, st); break;
        default: launch_q8_g<MT, P, DOTS, 5, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, nsplit, st); break;
    }
}

template <int MT, int P, bool DOTS, int GPW, int TPW = 1>
static void launch_q4_g(const void* W, const void* act, float* y, int32_t* dots, uint32_t M, uint32_t N, uint32_t K,
                        uint32_t ldy, int accumulate, uint32_t nw, hipStream_t st) {
    const ActLayout L = act_layout(EC_Q4_K, P * M, K);
    const uint32_t nT = round_up(N, 16) / 16, nB = L.Kp / 256;
    const uint32_t wave_floats = 2 * 8 * GPW * slots<MT>() + GPW * 256 * lrows<MT, P>() / 4;
    nw = min(nw, lds_cap_waves(wave_floats, TPW));
    const size_t lds = ((size_t)TPW * nw * 256 + (size_t)nw * wave_floats) * sizeof(float);
    hipLaunchKernelGGL((k_mv_q4_K<MT, P, DOTS, GPW, TPW>), dim3((nT + TPW - 1) / TPW), dim3(64 * nw), lds, st,
                       (const uint8_t*)W, (const uint8_t*)act, y, dots, M, N, K, nB, (uint32_t)L.xd_off,
                       (uint32_t)L.dxs_off, ldy, accumulate);
}

// M = 1 with one piece: the activation operand by row broadcasts instead of
// LDS staging (k_mv_q4_K_m1; EC_MV_Q4_M1=staged selects k_mv_q4_K, for
// comparison).
static bool q4_m1_direct() {
    static bool v = [] {
        const char* e = getenv("EC_MV_Q4_M1");
        return !(e && strcmp(e, "staged") == 0);
    }();
    return v;
}

template <int MT, int P, bool DOTS>
static void launch_q4(const void* W, const void* act, float* y, int32_t* dots, uint32_t M, uint32_t N, uint32_t K,
                      uint32_t ldy, int accumulate, hipStream_t st) {
    const uint32_t nT = round_up(N, 16) / 16, nB = round_up(K, 256) / 256;
    int gpw;
    uint32_t nw;
    plan(nT, nB, MT == 1 ? 3 : 1, gpw, nw, target_waves_q4());
    if constexpr (MT == 1 && P == 1 && !DOTS) {
        if (q4_m1_direct()) {
            const ActLayout L = act_layout(EC_Q4_K, 1, K);
            const size_t lds = (size_t)nw * 16 * sizeof(float);
            switch (gpw) {
#define EC_Q4M1(G)                                                                                          \
    hipLaunchKernelGGL((k_mv_q4_K_m1<G>), dim3(nT), dim3(64 * nw), lds, st, (const uint8_t*)W, (const uint8_t*)act, \
                       y, N, nB, (uint32_t)L.xd_off, (uint32_t)L.dxs_off, accumulate);                   \
    break;
                case 1: EC_Q4M1(1)
                case 2: EC_Q4M1(2)
                default: EC_Q4M1(3)
#undef EC_Q4M1
            }
            return;
        }
    }
    // M = 8 with two pieces and M = 16: two 16-row tiles per wave (each staged
    // activation super-block serves both) while that leaves >= 128
    // workgroups (EC_MV_TPW_Q4=1 keeps one; the other M and piece counts
    // spill registers with two tiles)
    if constexpr (((MT == 8 && P == 2) || MT == 16) && !DOTS) {
        if (tpw_q4() == 2 && (nT + 1) / 2 >= 128 && gpw == 1) {
            launch_q4_g<MT, P, DOTS, 1, 2>(W, act, y, dots, M, N, K, ldy, accumulate, nw, st);
            return;
        }
    }
    if constexpr (MT > 1) {  // the plan gives M > 1 one super-block per pass
        launch_q4_g<MT, P, DOTS, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, st);
    } else {
        switch (gpw) {
            case 1: launch_q4_g<MT, P, DOTS, 1>(W, act, y, dots, M, N, K, ldy, accumulate, nw, st); break;
            case 2: launch_q4_g<MT, P, DOTS, 2>(W, act, y, dots, M, N, K, ldy, accumulate, nw, st); break;
            default: launch_q4_g<MT, P, DOTS, 3>(W, act, y, dots, M, N, K, ldy, accumulate, nw, st); break;
        }
    }
}

template <int P, bool DOTS>
static void dispatch_p(int fmt, const void* W, const void* act, float* y, int32_t* dots, uint32_t M, uint32_t N,
                       uint32_t K, uint32_t ldy, int accumulate, hipStream_t st, uint32_t nsplit) {
    if (fmt == EC_Q8_0) {
        if (M == 1) launch_q8<1, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st, nsplit);
        else if (M <= 4) launch_q8<4, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st, nsplit);
        else if (M <= 8) launch_q8<8, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st, nsplit);
        else launch_q8<16, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st, nsplit);
    } else {
        if (M == 1) launch_q4<1, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st);
        else if (M <= 4) launch_q4<4, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st);
        else if (M <= 8) launch_q4<8, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st);
        else launch_q4<16, P, DOTS>(W, act, y, dots, M, N, K, ldy, accumulate, st);
    }
}

template <bool DOTS>
static int dispatch(int fmt, uint32_t pieces, const void* W, const void* act, float* y, int32_t* dots, uint32_t M,
                    uint32_t N, uint32_t K, uint32_t ldy, int accumulate, hipStream_t st, uint32_t nsplit = 1) {
    if (pieces == 2) dispatch_p<2, DOTS>(fmt, W, act, y, dots, M, N, K, ldy, accumulate, st, nsplit);
    else dispatch_p<1, DOTS>(fmt, W, act, y, dots, M, N, K, ldy, accumulate, st, nsplit);
    return EC_OK;
}

// Plain streaming read (HBM bandwidth calibration): each thread sums 16-byte
// loads with a grid stride (nothing is written unless a checksum hits a magic value).
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ src, size_t n16, uint32_t* out) {
    uint32_t acc = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;  // keeps the loads live; practically never taken
}

// The same read with a chosen launch shape: U non-temporal 16-byte loads in
// flight per thread per step (the single-launch read ceiling sweep).
template <int U>
__global__ __launch_bounds__(1024) void k_stream_read_u(const uint8_t* __restrict__ src, size_t n16, uint32_t* out) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i0 = (size_t)blockIdx.x * blockDim.x * U + threadIdx.x; i0 < n16; i0 += stride * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = i0 + (size_t)u * blockDim.x;
            v[u] = i < n16 ? ld_stream16(src + 16 * i) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

}  // namespace ec

using namespace ec;

extern "C" int ec_stream_read(const void* src, size_t bytes, uint32_t* out, uint32_t blocks, void* stream) {
    if (!src || !out || bytes % 16 || blocks == 0) return ec_set_error(EC_ERR_ARG, "ec_stream_read: bad argument");
    hipLaunchKernelGGL(k_stream_read, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src, bytes / 16,
                       out);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_stream_read_shape(const void* src, size_t bytes, uint32_t* out, uint32_t blocks, uint32_t threads,
                                    uint32_t unroll, void* stream) {
    if (!src || !out || bytes % 16 || blocks == 0 || (threads != 256 && threads != 512 && threads != 1024))
        return ec_set_error(EC_ERR_ARG, "ec_stream_read_shape: bad argument");
    const uint8_t* s = (const uint8_t*)src;
    hipStream_t st = (hipStream_t)stream;
    switch (unroll) {
        case 1: hipLaunchKernelGGL(k_stream_read_u<1>, dim3(blocks), dim3(threads), 0, st, s, bytes / 16, out); break;
        case 2: hipLaunchKernelGGL(k_stream_read_u<2>, dim3(blocks), dim3(threads), 0, st, s, bytes / 16, out); break;
        case 4: hipLaunchKernelGGL(k_stream_read_u<4>, dim3(blocks), dim3(threads), 0, st, s, bytes / 16, out); break;
        case 8: hipLaunchKernelGGL(k_stream_read_u<8>, dim3(blocks), dim3(threads), 0, st, s, bytes / 16, out); break;
        default: return ec_set_error(EC_ERR_ARG, "ec_stream_read_shape: unroll must be 1, 2, 4 or 8");
    }
    EC_CHECK_LAUNCH();
    return EC_OK;
}

static int check_mv(int fmt, uint32_t pieces, const void* W, const void* act, const void* out, uint32_t M,
                    uint32_t N, uint32_t K, const char* who) {
    if (fmt != EC_Q8_0 && fmt != EC_Q4_K) return ec_set_error(EC_ERR_UNSUPPORTED, "matvec: format must be Q8_0 or Q4_K");
    if (!W || !act || !out || M == 0 || M > 16 || N == 0 || K == 0 || K % (fmt == EC_Q8_0 ? 32u : 256u) ||
        (pieces != 1 && pieces != 2)) {
        char buf[192];
        snprintf(buf, sizeof buf, "%s: bad arguments (M=%u N=%u K=%u pieces=%u; need 1<=M<=16, K%%%u==0, 1 or 2 pieces)",
                 who, M, N, K, pieces, fmt == EC_Q8_0 ? 32u : 256u);
        return ec_set_error(EC_ERR_ARG, buf);
    }
    return EC_OK;
}

extern "C" int ec_matvec_pieces(int fmt, uint32_t pieces, const void* tiled, const void* act, float* y, uint32_t M,
                                uint32_t N, uint32_t K, uint32_t ldy, int accumulate, void* stream) {
    int rc = check_mv(fmt, pieces, tiled, act, y, M, N, K, "ec_matvec");
    if (rc) return rc;
    if (ldy < N) return ec_set_error(EC_ERR_ARG, "ec_matvec: ldy < N");
    dispatch<false>(fmt, pieces, tiled, act, y, nullptr, M, N, K, ldy, accumulate, (hipStream_t)stream);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_matvec(int fmt, const void* tiled, const void* act, float* y, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t ldy, int accumulate, void* stream) {
    return ec_matvec_pieces(fmt, 1, tiled, act, y, M, N, K, ldy, accumulate, stream);
}

extern "C" int ec_matvec_split_pieces(int fmt, uint32_t pieces, const void* tiled, const void* act, float* parts,
                                      uint32_t M, uint32_t N, uint32_t K, uint32_t nsplit, void* stream) {
    int rc = check_mv(fmt, pieces, tiled, act, parts, M, N, K, "ec_matvec_split");
    if (rc) return rc;
    if (fmt != EC_Q8_0) return ec_set_error(EC_ERR_UNSUPPORTED, "ec_matvec_split: Q8_0 weights only");
    if (nsplit == 0 || nsplit > round_up(K, 128) / 128)
        return ec_set_error(EC_ERR_ARG, "ec_matvec_split: nsplit must be in [1, ceil(K/128)]");
    dispatch<false>(fmt, pieces, tiled, act, parts, nullptr, M, N, K, N, 0, (hipStream_t)stream, nsplit);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_matvec_split(int fmt, const void* tiled, const void* act, float* parts, uint32_t M, uint32_t N,
                               uint32_t K, uint32_t nsplit, void* stream) {
    return ec_matvec_split_pieces(fmt, 1, tiled, act, parts, M, N, K, nsplit, stream);
}

extern "C" int ec_block_dots_pieces(int fmt, uint32_t pieces, const void* tiled, const void* act, int32_t* out,
                                    uint32_t M, uint32_t N, uint32_t K, void* stream) {
    int rc = check_mv(fmt, pieces, tiled, act, out, M, N, K, "ec_block_dots");
    if (rc) return rc;
    dispatch<true>(fmt, pieces, tiled, act, nullptr, out, M, N, K, N, 0, (hipStream_t)stream);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_block_dots(int fmt, const void* tiled, const void* act, int32_t* out, uint32_t M, uint32_t N,
                             uint32_t K, void* stream) {
    return ec_block_dots_pieces(fmt, 1, tiled, act, out, M, N, K, stream);
}

extern "C" int ec_matvec_gguf_f32(int fmt, const void* gguf, const float* x, float* y, uint32_t M, uint32_t K,
                                  void* stream) {
    if (M == 0) return EC_OK;
    if (!gguf || !x || !y) return ec_set_error(EC_ERR_ARG, "ec_matvec_gguf_f32: null pointer");
    if (fmt != EC_Q8_0 && fmt != EC_Q4_K && fmt != EC_Q2_K && fmt != EC_F16)
        return ec_set_error(EC_ERR_UNSUPPORTED, "ec_matvec_gguf_f32: unsupported format");
    // Q8_0 / Q4_K weight stream (gguf_mv.hip) where the shape allows it
    if (gguf_mv_fast(fmt, (const uint8_t*)gguf, x, y, M, K, (hipStream_t)stream) == EC_OK) {
        EC_CHECK_LAUNCH();
        return EC_OK;
    }
    hipLaunchKernelGGL(k_matvec_gguf_f32, dim3(M), dim3(64), 0, (hipStream_t)stream, fmt, (const uint8_t*)gguf, x, y,
                       M, K);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_dequant_dot_int8(const float* q, const int8_t* keys, const float* scales, float* scores,
                                   uint32_t dim, uint32_t seq_len, void* stream) {
    if (seq_len == 0) return EC_OK;
    if (!q || !keys || !scales || !scores) return ec_set_error(EC_ERR_ARG, "ec_dequant_dot_int8: null pointer");
    hipLaunchKernelGGL(k_dequant_dot_int8, dim3(seq_len), dim3(64), 0, (hipStream_t)stream, q, keys, scales, scores,
                       dim, seq_len);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_dequantize_to_fp16(int fmt, const void* src, uint16_t* dst, size_t n_weights, void* stream) {
    size_t per = fmt == EC_Q8_0 ? 32 : 256;
    if (fmt != EC_Q8_0 && fmt != EC_Q4_K && fmt != EC_Q2_K)
        return ec_set_error(EC_ERR_UNSUPPORTED, "ec_dequantize_to_fp16: unsupported format");
    size_t nblk = n_weights / per;
    if (nblk == 0) return EC_OK;
    if (!src || !dst) return ec_set_error(EC_ERR_ARG, "ec_dequantize_to_fp16: null pointer");
    hipLaunchKernelGGL(k_dequant_fp16, dim3((nblk + 127) / 128), dim3(128), 0, (hipStream_t)stream, fmt,
                       (const uint8_t*)src, dst, nblk);
    EC_CHECK_LAUNCH();
    return EC_OK;
}
