// attention_prefill.hip — causal INT8 attention of a prompt chunk (gfx950).
//
// Query token t of the chunk sits at position pos0 + t and attends over cache
// positions 0 .. pos0 + t of its sequence (the chunk's own K/V rows are
// appended first), per head exactly the decode attention of
// echo-core-zig/src/inference/engine.zig:563-616: q head h reads kv head
// h % n_kv, s_p = q.K_p * ks_p / sqrt(256), softmax, o = sum_p a_p V_p vs_p.
//
// One workgroup serves QB = 32/G query tokens x the G query heads of one kv
// head (32 query rows) and walks the key blocks of 64 positions up to its last
// token once: each block's K and V bytes are staged in LDS a single time for
// all 32 rows (V transposed to [dim][position]).  Scores and softmax . V run
// on v_mfma_i32_16x16x32_i8 as in the decode kernel: q and (probability x V
// row scale) are each split into three int8 pieces (layout.hpp split_pieces),
// so every product is an exact int32 and the pieces recombine in fp32.  The
// A rows of a 16-row MFMA tile are 4 query rows x 4 piece slots (the fourth
// zero), so the lanes of one DPP row hold one query row's scores, running
// max / sum and output: the online softmax needs no LDS.  Contraction
// indices are assigned so that each lane's share is contiguous (dims 64g ..
// 64g+63, positions 16g .. 16g+15 for lane group g), fetched with 16-byte
// LDS reads.
#include "common.hpp"
#include "layout.hpp"

namespace ec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr uint32_t kHd = 256;         // head_dim
constexpr uint32_t kKb = 64;          // key positions per block
constexpr uint32_t kRows = 32;        // query rows (token x head) per workgroup
constexpr uint32_t kKs = kHd + 16;    // LDS bytes per staged K row
constexpr uint32_t kVs = kKb / 4 + 2; // LDS dwords per V^T row (8-byte aligned, conflict-free b64 reads)
// V^T row d starts at dword d*kVs + 2*(d/16): without the skew the 16 rows a
// store instruction writes (dims 16*dg + const, dg = 0..15) would all start
// in the same bank (16*kVs is a multiple of the 32 banks), a 16-way conflict
// (512 tokens at 3584: 291 -> 249 us)
__device__ __forceinline__ uint32_t vt_at(uint32_t d, uint32_t col) { return d * kVs + 2 * (d >> 4) + col; }
constexpr uint32_t kPs = kKb + 8;     // LDS bytes per probability row
// blocks between forced flushes of the int32 softmax . V accumulators:
// |acc| <= 64 * kFlushBlocks * 127 * 127 < 2^31
constexpr uint32_t kFlushBlocks = 2048;
// the walk is cut into segments of about kSegBlocks key blocks (at most
// kMaxSegments), each its own workgroup, merged by k_attn_prefill_merge:
// floats per partial row = 256 outputs + max + sum
constexpr uint32_t kSegBlocks = 16, kMaxSegments = 8, kPartStride = kHd + 2;
// segments only while the (query block, kv head) workgroups number fewer
// than this (one per CU): with one workgroup per CU already, splitting only
// adds work (512 tokens at 3584: 249 us unsplit, 298 us in 4 segments; 128
// tokens at 3968: 227 -> 77 us in 4 segments)
constexpr uint64_t kSplitBelow = 256;
__host__ __device__ inline uint32_t prefill_segments(uint32_t positions) {
    const uint32_t nkb = (positions + kKb - 1) / kKb;
    const uint32_t s = (nkb + kSegBlocks - 1) / kSegBlocks;
    return s < 1 ? 1 : (s > kMaxSegments ? kMaxSegments : s);
}

struct PrefillLds {
    uint8_t K[kKb][kKs];
    uint32_t vT[kHd * kVs + 2 * (kHd / 16)];  // [dim][position quad], rows skewed (vt_at)
    uint8_t P[kRows / 4][16][kPs];    // per row tile: [4 query rows x 4 piece slots][position]
    uint8_t q[kRows][kQPieces][kHd];  // q pieces of the workgroup's query rows
    float qs[kRows][4];               // piece steps (slot 3 unused)
    float ks[kKb], vs[kKb];
    float vsw[4];  // per-wave maxima of the V row scales
};

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | (uint64_t)lo); }

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, lane_xor<1>(v));
    v = fmaxf(v, lane_xor<2>(v));
    v = fmaxf(v, lane_xor<4>(v));
    v = fmaxf(v, lane_xor<8>(v));
    return v;
}

}  // namespace

// grid 8 * ceil(nqb * n_kv / 8) (nqb = ceil(T / (32/G)) query blocks), block
// 256.  Workgroups are dispatched to the 8 XCDs round-robin (blockIdx % 8);
// XCD x takes the contiguous (kv head, query block) range [x*per, (x+1)*per)
// in kv-head-major order, so each XCD's L2 holds the K/V rows of one or two
// kv heads instead of all of them (every query block re-reads its kv head's
// cache).  Query row r (0 .. 31) is token r/G of the workgroup's QB tokens
// and head kvh + n_kv*(r%G); row tile i (8 of them) holds query rows
// 4i .. 4i+3, wave w owns tiles 2w and 2w+1.
template <int G>
__global__ __launch_bounds__(256) void k_attn_prefill(const float* __restrict__ q, const int8_t* __restrict__ keys,
                                                      const int8_t* __restrict__ vals,
                                                      const float* __restrict__ kscales,
                                                      const float* __restrict__ vscales, float* __restrict__ out,
                                                      float* __restrict__ part, uint32_t T, uint32_t pos0,
                                                      uint32_t n_kv, uint32_t S) {
    constexpr uint32_t QB = kRows / G;  // query tokens per workgroup
    __shared__ __align__(16) PrefillLds L;  // 16-byte aligned: b128 / b64 LDS accesses
    const uint32_t nqb = (T + QB - 1) / QB, total = nqb * n_kv * S, per = (total + 7) / 8;
    const uint32_t wg = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (wg >= total) return;  // grid padding (whole workgroup, before any barrier)
    const uint32_t kvh = wg / (nqb * S), qb = (wg / S) % nqb, seg = wg % S;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const uint32_t n_heads = n_kv * G;
    const uint32_t t_first = qb * QB, n_tok = min(QB, T - t_first);
    const uint32_t last_pos = pos0 + t_first + n_tok - 1;
    const uint32_t nkb = last_pos / kKb + 1;
    // segment seg of S of the walk: key blocks [kb0, kb1) (possibly empty)
    const uint32_t kb0 = seg * nkb / S, kb1 = (seg + 1) * nkb / S;
    const size_t row = (size_t)n_kv * kHd;
    const int8_t* kb = keys + (size_t)kvh * kHd;
    const int8_t* vb = vals + (size_t)kvh * kHd;

    // ---- q pieces of the 32 rows: wave w packs rows 8w .. 8w+7, lane = 4 dims
    for (uint32_t r = 8 * w; r < 8 * w + 8; ++r) {
        const uint32_t tq = r / G, head = kvh + n_kv * (r % G);
        float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tq < n_tok) v4 = *(const float4*)(q + ((size_t)(t_first + tq) * n_heads + head) * kHd + 4 * lane);
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
        float amax = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
        amax = wave_max(amax);
        uint32_t pw[kQPieces] = {0u, 0u, 0u};
        float steps[kQPieces];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int8_t pcs[kQPieces];
            split_pieces(vv[e], amax, pcs, steps);
#pragma unroll
            for (uint32_t pc = 0; pc < kQPieces; ++pc) pw[pc] |= (uint32_t)(uint8_t)pcs[pc] << (8 * e);
        }
#pragma unroll
        for (uint32_t pc = 0; pc < kQPieces; ++pc) *(uint32_t*)&L.q[r][pc][4 * lane] = pw[pc];
        if (lane == 0) *(float4*)&L.qs[r][0] = make_float4(steps[0], steps[1], steps[2], 0.f);
    }

    // ---- staging of key block b: K rows (thread = 16 bytes of one row) and V
    // transposed (thread = 16 dims x positions kq, kq+16, kq+32, kq+48 of the
    // block, 4x4 byte transposes): softmax . V contracts over the index
    // 4*(position % 16) + position / 16, so that a lane's four probabilities
    // (its position in each 16-position key tile) form one LDS dword.
    // Positions past last_pos repeat last_pos (masked in the scores).
    u32x4 kr[4], vr[4];
    float ksr = 0.f, vsr = 0.f;
    auto load = [&](uint32_t b) {
        const uint32_t p0 = b * kKb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = tid + 256 * j, key = i / 16, c = i % 16;
            const uint32_t p = min(p0 + key, last_pos);
            kr[j] = *(const u32x4*)(kb + (size_t)p * row + 16 * c);
        }
        const uint32_t dg = tid % 16, kq = tid / 16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t p = min(p0 + kq + 16 * j, last_pos);
            vr[j] = *(const u32x4*)(vb + (size_t)p * row + 16 * dg);
        }
        if (tid < kKb) {
            const uint32_t p = min(p0 + tid, last_pos);
            ksr = kscales[(size_t)p * n_kv + kvh];
            vsr = vscales[(size_t)p * n_kv + kvh];
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = tid + 256 * j, key = i / 16, c = i % 16;
            *(u32x4*)&L.K[key][16 * c] = kr[j];
        }
        const uint32_t dg = tid % 16, kq = tid / 16;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t w0 = vr[0][c], w1 = vr[1][c], w2 = vr[2][c], w3 = vr[3][c];
            const uint32_t a0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u), a1 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);
            const uint32_t b0 = __builtin_amdgcn_perm(w3, w2, 0x05010400u), b1 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
            L.vT[vt_at(16 * dg + 4 * c + 0, kq)] = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
            L.vT[vt_at(16 * dg + 4 * c + 1, kq)] = __builtin_amdgcn_perm(b0, a0, 0x07060302u);
            L.vT[vt_at(16 * dg + 4 * c + 2, kq)] = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
            L.vT[vt_at(16 * dg + 4 * c + 3, kq)] = __builtin_amdgcn_perm(b1, a1, 0x07060302u);
        }
        if (tid < kKb) {
            L.ks[tid] = ksr;
            L.vs[tid] = vsr;
        }
    };

    if (kb0 < kb1) load(kb0);
    // piece slot 3 of every probability row stays zero
    for (uint32_t i = tid; i < sizeof(L.P) / 4; i += 256) ((uint32_t*)&L.P[0][0][0])[i] = 0u;
    __syncthreads();  // q pieces and the zero rows complete

    // per owned tile tt (tile 2w + tt): A operand (lane (r, g): piece r%4 of
    // query row 4i + r/4, dims 64g .. 64g+63; piece slot 3 is zero) and the
    // lane's query row 4i + g in the D layout with its softmax state
    u32x4 qa[2][4];
    uint32_t my_tq[2], my_head[2], my_pos[2];
    float qs[2][3], m[2], l[2], o[2][16];
    v4i acc[2][16];  // softmax . V since the last flush, int32 per piece (rows 4*g4 + piece)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const uint32_t i = 2 * w + tt, ar = 4 * i + r16 / 4, pc = r16 % 4;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            qa[tt][c] = pc < kQPieces ? *(const u32x4*)&L.q[ar][pc][64 * g4 + 16 * c] : u32x4{0u, 0u, 0u, 0u};
        const uint32_t mr = 4 * i + g4;
        my_tq[tt] = mr / G;
        my_head[tt] = kvh + n_kv * (mr % G);
        my_pos[tt] = pos0 + t_first + my_tq[tt];
#pragma unroll
        for (int pc2 = 0; pc2 < 3; ++pc2) qs[tt][pc2] = L.qs[mr][pc2];
        m[tt] = -INFINITY;
        l[tt] = 0.f;
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            o[tt][d] = 0.f;
            acc[tt][d] = v4i{0, 0, 0, 0};
        }
    }
    constexpr float scale = 1.0f / 16.0f;  // 1/sqrt(256)
    // fixed piece steps for the whole walk: p = e * vs <= vs_max (e <= 1
    // against the row's running maximum m)
    float vmax;
    {
        float v = 0.0f;
        const uint32_t pend = min(kb1 * kKb, last_pos + 1);
        for (uint32_t p = kb0 * kKb + tid; p < pend; p += 256) v = fmaxf(v, vscales[(size_t)p * n_kv + kvh]);
        v = wave_max(v);
        if (lane == 0) L.vsw[w] = v;
        __syncthreads();
        vmax = fmaxf(fmaxf(L.vsw[0], L.vsw[1]), fmaxf(L.vsw[2], L.vsw[3]));
    }
    const float st0 = vmax > 0.0f ? vmax * (1.0f / 127.0f) : 1.0f, iv0 = vmax > 0.0f ? 127.0f / vmax : 1.0f;
    const float st1 = st0 * (1.0f / 254.0f), iv1 = iv0 * 254.0f;
    const float st2 = st1 * (1.0f / 254.0f), iv2 = iv1 * 254.0f;

    for (uint32_t b = kb0; b < kb1; ++b) {
        __syncthreads();  // the previous block's readers of K, vT are done
        store();
        __syncthreads();
        if (b + 1 < kb1) load(b + 1);
        // ---- scores of both owned tiles: 4 key tiles x 8 k-steps each; K
        // operand lane (r, g) = position 16kt + r, dims 64g .. 64g+63
        // (one key tile's K operand at a time: 16 VGPRs instead of 64)
        v4i C[2][4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            u32x4 kb[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) kb[c] = *(const u32x4*)&L.K[16 * kt + r16][64 * g4 + 16 * c];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                C[tt][kt] = v4i{0, 0, 0, 0};
#pragma unroll
                for (int m8 = 0; m8 < 8; ++m8) {
                    const u32x4 a = qa[tt][m8 / 2], bb = kb[m8 / 2];
                    const long A = (m8 & 1) ? pack2(a.z, a.w) : pack2(a.x, a.y);
                    const long B = (m8 & 1) ? pack2(bb.z, bb.w) : pack2(bb.x, bb.y);
                    C[tt][kt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, C[tt][kt], 0, 0, 0);
                }
            }
        }
        // ---- softmax against the running row maximum m; lane (r16 = position
        // in key tile, g4 = query row).  When a row's maximum rises (or every
        // kFlushBlocks blocks, the int32 bound) the wave flushes: o = (o +
        // sum_j step_j * acc_j) * exp(m_old - m_new), acc = 0, l rescaled.
        // Otherwise probabilities keep the fixed steps and softmax . V
        // accumulates in the MFMA's int32 registers with no fp32 epilogue.
        float sc[2][4], bm[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            bm[tt] = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const uint32_t kp = b * kKb + 16 * kt + r16;
                const v4i c4 = C[tt][kt];
                const float raw = (qs[tt][0] * (float)c4[0] + qs[tt][1] * (float)c4[1]) + qs[tt][2] * (float)c4[2];
                sc[tt][kt] = kp <= my_pos[tt] ? raw * L.ks[16 * kt + r16] * scale : -INFINITY;
                bm[tt] = fmaxf(bm[tt], sc[tt][kt]);
            }
            bm[tt] = row16_max(bm[tt]);
        }
        if (__any(bm[0] > m[0] || bm[1] > m[1]) || ((b - kb0) % kFlushBlocks == 0 && b > kb0)) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                // -inf until a row sees a visible position (a later segment
                // may start past a row's own position)
                const float mn = fmaxf(m[tt], bm[tt]);
                const float corr = mn == -INFINITY ? 1.0f : __expf(m[tt] - mn);  // first: exp(-inf) = 0
#pragma unroll
                for (int dt = 0; dt < 16; ++dt) {
                    const v4i c = acc[tt][dt];
                    o[tt][dt] = (o[tt][dt] + ((st0 * (float)c[0] + st1 * (float)c[1]) + st2 * (float)c[2])) * corr;
                    acc[tt][dt] = v4i{0, 0, 0, 0};
                }
                l[tt] *= corr;
                m[tt] = mn;
            }
        }
        // probability x V row scale as three int8 pieces (fixed steps): row
        // 4*g4 + piece of tile i; the four key tiles' values of position r16
        // are bytes 0..3 of dword r16 (contraction index 4*r16 + kt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const uint32_t i = 2 * w + tt;
            const float mu = m[tt] == -INFINITY ? 0.0f : m[tt];  // every score masked while m is -inf
            uint32_t pw[kQPieces] = {0u, 0u, 0u};
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const float e = __expf(sc[tt][kt] - mu);  // <= 1; masked: 0
                l[tt] += e;
                const float pr = e * L.vs[16 * kt + r16];
                const float q0 = fminf(rintf(pr * iv0), 127.0f);
                const float r1 = fmaf(-q0, st0, pr);
                const float q1 = fminf(fmaxf(rintf(r1 * iv1), -127.0f), 127.0f);
                const float r2 = fmaf(-q1, st1, r1);
                const float q2 = fminf(fmaxf(rintf(r2 * iv2), -127.0f), 127.0f);
                pw[0] |= (uint32_t)(uint8_t)(int8_t)q0 << (8 * kt);
                pw[1] |= (uint32_t)(uint8_t)(int8_t)q1 << (8 * kt);
                pw[2] |= (uint32_t)(uint8_t)(int8_t)q2 << (8 * kt);
            }
#pragma unroll
            for (uint32_t pc = 0; pc < kQPieces; ++pc) ((uint32_t*)&L.P[i][4 * g4 + pc][0])[r16] = pw[pc];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's P dwords are in LDS before its reads below
        __builtin_amdgcn_wave_barrier();
        // ---- P . V: 16 dim tiles x 2 k-steps per tile (lane group g4:
        // contraction indices 16g4 .. 16g4+15); each V operand serves both tiles
        long A[2][2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const uint2* ap = (const uint2*)&L.P[2 * w + tt][r16][16 * g4];
            const uint2 a0 = ap[0], a1 = ap[1];
            A[tt][0] = pack2(a0.x, a0.y);
            A[tt][1] = pack2(a1.x, a1.y);
        }
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
            const uint2* bp = (const uint2*)&L.vT[vt_at(16 * dt + r16, 4 * g4)];
            const uint2 b0 = bp[0], b1 = bp[1];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                acc[tt][dt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[tt][0], pack2(b0.x, b0.y), acc[tt][dt], 0, 0, 0);
                acc[tt][dt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[tt][1], pack2(b1.x, b1.y), acc[tt][dt], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const float lt = row16_sum(l[tt]);
        if (my_tq[tt] >= n_tok) continue;
        const size_t qi = (size_t)(t_first + my_tq[tt]) * n_heads + my_head[tt];
        if (S == 1) {  // the whole walk: normalized output
            const float inv = 1.0f / lt;
            float* dst = out + qi * kHd;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                const v4i c = acc[tt][dt];
                dst[16 * dt + r16] = (o[tt][dt] + ((st0 * (float)c[0] + st1 * (float)c[1]) + st2 * (float)c[2])) * inv;
            }
        } else {  // segment partial: unnormalized o, row maximum, row sum
            float* dst = part + ((size_t)seg * T * n_heads + qi) * kPartStride;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                const v4i c = acc[tt][dt];
                dst[16 * dt + r16] = o[tt][dt] + ((st0 * (float)c[0] + st1 * (float)c[1]) + st2 * (float)c[2]);
            }
            if (r16 == 0) {
                dst[kHd] = m[tt];
                dst[kHd + 1] = lt;
            }
        }
    }
}

// Combine the S segment partials of each (token, head): grid (T, n_heads),
// block 256 (one thread per dim).  A segment a row did not reach has m = -inf,
// l = 0 and weight 0.
__global__ __launch_bounds__(256) void k_attn_prefill_merge(const float* __restrict__ part, float* __restrict__ out,
                                                            uint32_t T, uint32_t n_heads, uint32_t S) {
    const size_t qi = (size_t)blockIdx.x * n_heads + blockIdx.y;
    const uint32_t d = threadIdx.x;
    const size_t seg_stride = (size_t)T * n_heads * kPartStride;
    const float* p = part + qi * kPartStride;
    float M = -INFINITY;
    for (uint32_t s = 0; s < S; ++s) M = fmaxf(M, p[s * seg_stride + kHd]);
    float o = 0.0f, l = 0.0f;
    for (uint32_t s = 0; s < S; ++s) {
        const float* ps = p + s * seg_stride;
        const float ms = ps[kHd];
        const float wgt = ms == -INFINITY ? 0.0f : __expf(ms - M);
        o = fmaf(wgt, ps[d], o);
        l = fmaf(wgt, ps[kHd + 1], l);
    }
    out[qi * kHd + d] = o / l;
}

}  // namespace ec

using namespace ec;

extern "C" size_t ec_attn_prefill_ws_bytes(uint32_t T, uint32_t n_heads, uint32_t max_ctx) {
    const uint32_t S = prefill_segments(max_ctx);
    return S > 1 ? (size_t)S * T * n_heads * kPartStride * sizeof(float) : 0;
}

extern "C" int ec_attn_prefill(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                               const float* vscales, float* out, uint32_t T, int32_t pos0, uint32_t n_heads,
                               uint32_t n_kv, uint32_t head_dim, uint32_t max_ctx, void* ws, void* stream) {
    if (T == 0) return EC_OK;
    if (!q || !keys || !vals || !kscales || !vscales || !out || head_dim != kHd || n_kv == 0 || n_heads % n_kv ||
        pos0 < 0 || (uint64_t)pos0 + T > max_ctx)
        return ec_set_error(EC_ERR_ARG, "ec_attn_prefill: need head_dim 256, n_heads % n_kv == 0, pos0 + T <= max_ctx");
    const uint32_t G = n_heads / n_kv;
    const hipStream_t st = (hipStream_t)stream;
    // segments: from the positions of this call, never more than the workspace
    // (sized for max_ctx) holds; no workspace: one segment
    const uint64_t blocks = (uint64_t)((T + 32 / G - 1) / (32 / G)) * n_kv;
    uint32_t S = 1;
    if (ws && blocks < kSplitBelow) {
        S = prefill_segments((uint32_t)pos0 + T);
        while (S > 1 && blocks * (S - 1) >= kSplitBelow) --S;  // enough workgroups with fewer segments
    }
    const uint64_t total = blocks * S;
    if (total > (1u << 28)) return ec_set_error(EC_ERR_ARG, "ec_attn_prefill: too many query blocks");
    const dim3 grid(8 * (uint32_t)((total + 7) / 8));
    float* part = (float*)ws;
    switch (G) {
        case 1:
            hipLaunchKernelGGL(k_attn_prefill<1>, grid, dim3(256), 0, st, q, keys, vals, kscales, vscales, out, part, T,
                               (uint32_t)pos0, n_kv, S);
            break;
        case 2:
            hipLaunchKernelGGL(k_attn_prefill<2>, grid, dim3(256), 0, st, q, keys, vals, kscales, vscales, out, part, T,
                               (uint32_t)pos0, n_kv, S);
            break;
        case 4:
            hipLaunchKernelGGL(k_attn_prefill<4>, grid, dim3(256), 0, st, q, keys, vals, kscales, vscales, out, part, T,
                               (uint32_t)pos0, n_kv, S);
            break;
        default:
            return ec_set_error(EC_ERR_UNSUPPORTED, "ec_attn_prefill: n_heads / n_kv must be 1, 2 or 4");
    }
    EC_CHECK_LAUNCH();
    if (S > 1) {
        hipLaunchKernelGGL(k_attn_prefill_merge, dim3(T, n_heads), dim3(256), 0, st, part, out, T, n_heads, S);
        EC_CHECK_LAUNCH();
    }
    return EC_OK;
}
