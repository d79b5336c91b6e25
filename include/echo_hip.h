/*
 * echo_hip.h — the C ABI of libechohip.so, echo-core's decode hot path on
 * AMD Instinct MI355X (gfx950).
 *
 * Every entry point takes DEVICE pointers (hipMalloc'd or managed), sizes and
 * a hipStream_t passed as void* (NULL = the null stream), is stream-ordered and
 * returns an ec_status (0 = success).  Nothing here allocates except where a
 * function says so.  ec_last_error() returns a thread-local message for the
 * last failure.  The reference-signature wrappers (include/kernels/quant.h,
 * include/kernels/matvec.h, include/kv_cache.h, include/inference.h) are
 * built on these.
 *
 * Reference correspondence (paths relative to the echo-core source tree):
 *   ec_quantize_rows       src/kernels/quant.cpp:18-98  quantize_per_token_symmetric
 *   ec_matvec_q8_0         src/kernels/matvec.cpp:62-87 matvec_q8_0 (y += W x), M tokens at once
 *   ec_matvec_q4_K         src/kernels/matvec.cpp:92-142 matvec_q4_K
 *   ec_kv_append           src/kv_cache.cpp:89-113 KVCache::append
 *   ec_attn_decode         src/inference.cpp:330-405, echo-core-zig/src/inference/engine.zig:563-616
 *   ec_deltanet            echo-core-zig/src/kernels/qwen_linear.zig:207-250
 */
#ifndef ECHO_HIP_H
#define ECHO_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ec_status {
    EC_OK = 0,
    EC_ERR_ARG = 1,      /* bad size, alignment or null pointer */
    EC_ERR_HIP = 2,      /* a HIP runtime call failed */
    EC_ERR_UNSUPPORTED = 3,
};

/* Weight formats, numbered as the reference's GGMLType (include/gguf_reader.h:13-41). */
enum ec_wfmt { EC_F32 = 0, EC_F16 = 1, EC_Q8_0 = 6, EC_Q2_K = 8, EC_Q4_K = 10 };

const char* ec_last_error(void);
/* Empties this thread's last-error message (the reference-signature wrappers
 * return void, so a caller clears it before a call and reads it after). */
void ec_clear_error(void);
int ec_device_init(int device);
/* Synchronous copy between any two host / device buffers (direction from the
 * pointers), for callers without their own HIP runtime binding. */
int ec_copy(void* dst, const void* src, size_t bytes);

/* ------------------------------------------------------------------ quantizer
 * Reference per-row quantizer on device (bit-exact): scale = amax/127 (1 if the
 * row is all zero); elements of whole 8-chunks q = sat8(rne(x*(1/scale))), tail
 * elements q = clamp(round_half_away(x/scale), +-127). */
int ec_quantize_rows(const float* x, int8_t* q, float* scales, uint32_t rows, uint32_t width, void* stream);

/* ------------------------------------------------------- decode weight layout
 * Weights are uploaded in GGUF byte order and repacked once into a "tiled"
 * layout whose loads are 16-byte aligned and match the int8 MFMA operand
 * layout.  Rows are grouped in tiles of 16 (N padded to 16); K is padded to
 * 128 (Q8_0) or 256 (Q4_K) with zero blocks.  The repacked buffer holds the
 * same bytes per block as GGUF (34 B per Q8_0 block, 144 B per Q4_K block).
 * gguf: N rows of K/32*34 (Q8_0) or K/256*144 (Q4_K) bytes. */
size_t ec_tiled_bytes(int fmt, uint32_t N, uint32_t K);
int ec_repack(int fmt, const void* gguf, void* tiled, uint32_t N, uint32_t K, void* stream);
/* Inverse of ec_repack (Q8_0 or Q4_K): tiled -> GGUF rows. */
int ec_unpack_tiled(int fmt, const void* tiled, void* gguf, uint32_t N, uint32_t K, void* stream);

/* --------------------------------------------------- activation quantization
 * M (1..16) fp32 activation rows x[M][K] are quantized per 32-element block
 * with the reference quantizer and stored in the lane order the matvec reads.
 * Q8_0 blocks are 32 consecutive elements; Q4_K blocks are the 32 positions of
 * one Q4_K sub-block (so every int8 block meets one 6-bit scale/min pair).
 * K must be a multiple of 32; the buffer is padded like the weights. */
size_t ec_act_bytes(int fmt, uint32_t M, uint32_t K);
int ec_quantize_act(int fmt, const float* x, void* act, uint32_t M, uint32_t K, void* stream);
/* Two-piece activations (no counterpart in the reference, whose matvecs take
 * fp32 x, src/kernels/matvec.cpp:62-142): pieces = 2 stores, per block, piece
 * 0 = the reference quantizer's int8 q0 at scale s and piece 1 = the residual
 * x - s*q0 quantized with the scale s/256, q1 = sat8(rne((x - s*q0) * (256/s)))
 * (x ~ s*q0 + (s/256)*q1, |error| <= s/512: within ~2e-5 relative of the
 * fp32 matvec instead of ~5e-3 with one piece).  The M tokens occupy 2M rows
 * of the one-piece layout (token i's pieces in rows 2i, 2i+1;
 * ec_act_unpack_pieces reads them back), scales per token; Q4_K's sum
 * becomes s * (sum q0 + sum q1 / 256).  pieces = 1 is ec_quantize_act. */
size_t ec_act_bytes_pieces(int fmt, uint32_t M, uint32_t K, uint32_t pieces);
int ec_quantize_act_pieces(int fmt, const float* x, void* act, uint32_t M, uint32_t K, uint32_t pieces,
                           void* stream);
/* Read back the quantized activation in natural order: xq[M][K] int8 (block
 * grouping as above, i.e. Q4_K values in sub-block order) and xd[M][K/32]. */
int ec_act_unpack(int fmt, const void* act, int8_t* xq, float* xd, uint32_t M, uint32_t K, void* stream);
/* The same for `pieces` (1 or 2) pieces: xq[pieces*M][K] (row 2i + p = token
 * i, piece p), xd[M][K/32]. */
int ec_act_unpack_pieces(int fmt, uint32_t pieces, const void* act, int8_t* xq, float* xd, uint32_t M, uint32_t K,
                         void* stream);

/* ------------------------------------------------------- decode matvec / GEMV
 * y[m][n] (+)= sum_b d_w[n,b] * d_x[m,b] * isum[m,n,b] for M (1..16) token rows,
 * isum = exact int32 dot of one 32-element block (Q8_0), and for Q4_K
 * y += sum_sb d_x * (d*sc * isum - dmin*m * xsum).  accumulate != 0 adds into y
 * (the reference's y += W x), else y is overwritten.  y is [M][ldy] fp32. */
int ec_matvec(int fmt, const void* tiled, const void* act, float* y, uint32_t M, uint32_t N, uint32_t K,
              uint32_t ldy, int accumulate, void* stream);
/* Split-K form of ec_matvec for Q8_0 (no counterpart in the reference: the
 * decode step's output projections use it to fill the GPU when N is small).
 * The K range is cut into nsplit (1 .. ceil(K/128)) balanced ranges of
 * 128-element chunks; parts[sp][M][N] receives range sp's partial sums.
 * sum over sp of parts == ec_matvec's y up to fp32 summation order. */
int ec_matvec_split(int fmt, const void* tiled, const void* act, float* parts, uint32_t M, uint32_t N, uint32_t K,
                    uint32_t nsplit, void* stream);
/* The int32 block dots themselves: out[m][n][K/32] (parity contract). */
int ec_block_dots(int fmt, const void* tiled, const void* act, int32_t* out, uint32_t M, uint32_t N, uint32_t K,
                  void* stream);
/* The same three over an activation of 1 or 2 pieces (ec_quantize_act_pieces):
 * with two pieces each block dot is 256*isum0 + isum1 (exact int32) scaled by
 * d_w * d_x / 256; ec_block_dots_pieces writes the dots of every layout row,
 * out[pieces*M][N][K/32] (row 2i + p: token i, piece p). */
int ec_matvec_pieces(int fmt, uint32_t pieces, const void* tiled, const void* act, float* y, uint32_t M, uint32_t N,
                     uint32_t K, uint32_t ldy, int accumulate, void* stream);
int ec_matvec_split_pieces(int fmt, uint32_t pieces, const void* tiled, const void* act, float* parts, uint32_t M,
                           uint32_t N, uint32_t K, uint32_t nsplit, void* stream);
int ec_block_dots_pieces(int fmt, uint32_t pieces, const void* tiled, const void* act, int32_t* out, uint32_t M,
                         uint32_t N, uint32_t K, void* stream);

/* ------------------------------------------- reference-semantics fp32 matvec
 * y[m] += W[m,:] . x over GGUF bytes with fp32 activations (no activation
 * quantization), for the drop-in wrappers of include/kernels/matvec.h. */
int ec_matvec_gguf_f32(int fmt, const void* gguf, const float* x, float* y, uint32_t M, uint32_t K, void* stream);
/* scores[p] = sum_k K[p,k]*scale[p]*q[k] (src/kernels/quant.cpp:100-144). */
int ec_dequant_dot_int8(const float* q, const int8_t* keys, const float* scales, float* scores, uint32_t dim,
                        uint32_t seq_len, void* stream);
/* GGUF blocks -> fp16 (src/kernels/quant.cpp:308-396). */
int ec_dequantize_to_fp16(int fmt, const void* src, uint16_t* dst, size_t n_weights, void* stream);

/* ----------------------------------------------------------------- KV cache
 * Cache layout per layer (the reference's, include/kv_cache.h:7-19):
 * keys/vals int8 [max_seq][n_kv][head_dim], kscales/vscales fp32 [max_seq][n_kv].
 * ec_kv_append quantizes one token per sequence: k, v [n_seq][n_kv*head_dim];
 * sequence s writes position pos[s] of its own cache (cache base + s*seq_stride
 * elements for int8 arrays, s*seq_stride/head_dim for scales).  pos[s] < 0
 * skips the sequence.  One scale per (token, kv_head) row of head_dim. */
int ec_kv_append(const float* k, const float* v, int8_t* keys, int8_t* vals, float* kscales, float* vscales,
                 const int32_t* pos, uint32_t n_seq, uint64_t seq_stride, uint32_t n_kv, uint32_t head_dim,
                 void* stream);

/* ------------------------------------------------------------- prefill GEMM
 * Y[m][n] (+)= sum_k X[m][k] * W[n][k] for M tokens (any M; prefill chunks of
 * 512) on int8 MFMA.  ec_gemm_quantize_act quantizes X (fp32 [M][K], row
 * stride K) per 32-element block with the reference quantizer into the tiled
 * token layout of gemm.hip (Q4_K: per sub-block of the reference's position
 * order); W is the tiled weight of ec_repack.  Exact int32 block dots, fp32
 * scaling: Q8_0 Y += dx*dw*isum; Q4_K Y += dx*(d*sc*isum - dmin*m*xsum).
 * ldy >= N; accumulate != 0 adds to Y. */
size_t ec_gemm_act_bytes(int fmt, uint32_t M, uint32_t K);
int ec_gemm_quantize_act(int fmt, const float* x, void* act, uint32_t M, uint32_t K, void* stream);  /* x 16-byte aligned */
int ec_gemm(int fmt, const void* tiled, const void* act, float* y, uint32_t M, uint32_t N, uint32_t K, uint32_t ldy,
            int accumulate, void* stream);

/* ------------------------------------------------------- INT8 attention decode
 * out[s][h][:] = softmax_p(q[s][h].K[p, h%n_kv] * ks / sqrt(head_dim)) . V[p, h%n_kv] * vs
 * over p < ctx[s] (ctx[s] <= 0: output zeros).  q, out: [n_seq][n_heads*head_dim].
 * Split-K over the context: ws must hold ec_attn_ws_bytes(...) bytes.
 * head_dim 256 with n_heads/n_kv in {1,2,4} runs QK^T on int8 MFMA with q
 * split into three int8 pieces (|q - sum| <= max|q| * 6.1e-8); other shapes
 * (head_dim 64/128, 8 heads per kv head) run an fp32 VALU kernel. */
size_t ec_attn_ws_bytes(uint32_t n_seq, uint32_t n_heads, uint32_t head_dim, uint32_t max_ctx);
int ec_attn_decode(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                   const float* vscales, float* out, const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride,
                   uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_ctx, void* ws, void* stream);

/* ec_attn_decode without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is a fixed
 * device array of ec_attn_noalloc_max_bytes() = 16 MiB per GPU, held until
 * the process ends; calls needing more (ec_attn_ws_bytes(n_seq, n_heads,
 * head_dim, max_ctx) > 16 MiB, e.g. more than ~1M total context positions at
 * 16 heads) fail with EC_ERR_ARG.  Nothing in it needs to start at zero.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (different streams, or threads) race and must be serialized by the caller.
 * The array's device address is looked up by ec_device_init, or on the
 * first call on a device. */
size_t ec_attn_noalloc_max_bytes(void);
int ec_attn_decode_noalloc(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                           const float* vscales, float* out, const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride,
                           uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_ctx, void* stream);

/* Same computation from q already packed into the three-piece int8 layout
 * (ec_glue_qk_rope_append writes it; ec_attn_qa_bytes(n_seq, n_heads) bytes
 * plus n_seq*n_heads*3 fp32 scales), head_dim 256, n_heads/n_kv in {1,2,4}.
 * act_q8 != NULL additionally writes out[] quantized into the Q8_0 activation
 * layout of ec_quantize_act (n_seq <= 16, K = n_heads*256), ready for the
 * output projection. */
size_t ec_attn_qa_bytes(uint32_t n_seq, uint32_t n_heads);
int ec_attn_decode_packed(const void* q_packed, const float* q_scales, const int8_t* keys, const int8_t* vals,
                          const float* kscales, const float* vscales, float* out, void* act_q8, const int32_t* ctx,
                          uint32_t n_seq, uint64_t seq_stride, uint32_t n_heads, uint32_t n_kv, uint32_t max_ctx,
                          void* ws, void* stream);
/* ec_attn_decode_packed whose act_q8 holds `pieces` (1 or 2) pieces per
 * element (ec_quantize_act_pieces' layout). */
int ec_attn_decode_packed_pieces(const void* q_packed, const float* q_scales, const int8_t* keys, const int8_t* vals,
                                 const float* kscales, const float* vscales, float* out, void* act_q8,
                                 const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride, uint32_t n_heads,
                                 uint32_t n_kv, uint32_t max_ctx, uint32_t pieces, void* ws, void* stream);

/* Causal attention of a prompt chunk over one sequence's cache: query token t
 * (q, out: [T][n_heads][256]) sits at position pos0 + t and attends over
 * positions 0 .. pos0 + t of keys/vals/kscales/vscales (the layout above, the
 * chunk's rows already appended), each head as ec_attn_decode computes it.
 * One pass over the cache per group of 32/G query tokens and kv head, QK^T and
 * softmax . V on int8 MFMA; with a workspace (ws, ec_attn_prefill_ws_bytes(T',
 * n_heads, max_ctx) bytes for any T <= T') long walks are cut into up to 8
 * segments run in parallel and merged; ws NULL: one segment.  head_dim 256,
 * n_heads / n_kv in {1, 2, 4}, pos0 + T <= max_ctx.  No counterpart in the
 * reference (its prefill runs the decode attention token by token,
 * engine.zig:520-621). */
size_t ec_attn_prefill_ws_bytes(uint32_t T, uint32_t n_heads, uint32_t max_ctx);
int ec_attn_prefill(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                    const float* vscales, float* out, uint32_t T, int32_t pos0, uint32_t n_heads, uint32_t n_kv,
                    uint32_t head_dim, uint32_t max_ctx, void* ws, void* stream);

/* --------------------------------------------------------------- delta-net
 * Gated delta rule for T tokens of n_seq sequences (qwen_linear.zig:207-250):
 *   S <- decay*S; kv = S^T k; delta = (v - kv)*beta; S += k (x) delta; o = S^T q/sqrt(d_k)
 * state: [n_seq][n_v][d_v][d_k] fp32, i.e. each head's S stored TRANSPOSED
 * relative to the reference (S[v][k], one contiguous d_k column per value
 * channel).  q, k: [T][n_seq][n_k][d_k] (L2-normalised by the caller),
 * v, out: [T][n_seq][n_v][d_v]; decay, beta: [T][n_seq][n_v] (beta after the
 * sigmoid).  v-head h reads q/k head h/(n_v/n_k).  d_k must be 128 and d_v a
 * multiple of 16.  The state stays on chip across the T tokens. */
int ec_deltanet(float* state, const float* q, const float* k, const float* v, const float* decay, const float* beta,
                float* out, uint32_t T, uint32_t n_seq, uint32_t n_v, uint32_t n_k, uint32_t d_k, uint32_t d_v,
                const int32_t* seq_pos, void* stream);

/* The same recurrence for a prompt chunk, in chunks of 64 tokens (prefill):
 * per chunk the decay-weighted key Gram matrix gives U = (I + A)^{-1} B (V -
 * G K S0) by forward substitution, then O and the next state from the chunk's
 * start state with fp32 MFMA products; chunks run in order, heads and value
 * columns in parallel.  Equal to ec_deltanet up to fp32 rounding (a decay below
 * 1e-30 counts as 1e-30).  d_k = d_v = 128; ws holds
 * ec_deltanet_chunked_ws_bytes(T, n_seq, n_v) bytes. */
size_t ec_deltanet_chunked_ws_bytes(uint32_t T, uint32_t n_seq, uint32_t n_v);
int ec_deltanet_chunked(float* state, const float* q, const float* k, const float* v, const float* decay,
                        const float* beta, float* out, uint32_t T, uint32_t n_seq, uint32_t n_v, uint32_t n_k,
                        uint32_t d_k, uint32_t d_v, const int32_t* seq_pos, void* ws, void* stream);

/* One decode token of a delta-net block (qwen_linear.zig:182-257), fused:
 * conv + SiLU over the ring conv state (see ec_glue_conv_gates), q/k L2 norms,
 * decay/beta gates, the delta rule on state (layout of ec_deltanet, d_k = d_v
 * = 128), gated RMSNorm with norm_w[128] and z = proj[conv_dim + h*128 + i],
 * quantized into act (Q8_0 activation layout, M = n_seq <= 16, K = n_v*128).
 * proj rows [n_seq][Nin] hold q|k|v (conv_dim) | z (n_v*128) | alpha | beta.
 * Sequences with pos[s] < 0 are skipped (state, conv state and act untouched). */
int ec_delta_step(const float* proj, uint32_t Nin, float* conv_state, const float* conv_w, const float* a_log,
                  const float* dt_bias, const float* norm_w, float* state, void* act, const int32_t* pos,
                  uint32_t n_seq, uint32_t n_k, uint32_t n_v, uint32_t kern, void* stream);
/* ec_delta_step_split writing the gated-norm output as fp32 out[n_seq][n_v*128]
 * (when out != NULL) and/or quantized into act (when act != NULL). */
int ec_delta_step_out(const float* proj, uint32_t nparts, uint32_t Nin, float* conv_state, const float* conv_w,
                      const float* a_log, const float* dt_bias, const float* norm_w, float* state, void* act,
                      float* out, const int32_t* pos, uint32_t n_seq, uint32_t n_k, uint32_t n_v, uint32_t kern,
                      void* stream);
/* ec_delta_step_out with act in `pieces` (1 or 2) pieces (ec_quantize_act_pieces' layout). */
int ec_delta_step_out_pieces(const float* proj, uint32_t nparts, uint32_t Nin, float* conv_state, const float* conv_w,
                             const float* a_log, const float* dt_bias, const float* norm_w, float* state, void* act,
                             float* out, const int32_t* pos, uint32_t n_seq, uint32_t n_k, uint32_t n_v,
                             uint32_t kern, uint32_t pieces, void* stream);
/* seq_pos (may be NULL): sequence s is skipped entirely (state untouched, no
 * output written) when seq_pos[s] < 0. */
/* ec_delta_step with the input projection given as nparts (1..8) partial sums
 * proj[nparts][n_seq][Nin] (ec_matvec_split's output), added in part order. */
int ec_delta_step_split(const float* proj, uint32_t nparts, uint32_t Nin, float* conv_state, const float* conv_w,
                        const float* a_log, const float* dt_bias, const float* norm_w, float* state, void* act,
                        const int32_t* pos, uint32_t n_seq, uint32_t n_k, uint32_t n_v, uint32_t kern, void* stream);

/* ------------------------------------------------------------ decode-step glue
 * Fused per-token ops of the hybrid decoder (semantics in glue.hip); every
 * "_quant" op writes the Q8_0 activation layout consumed by ec_matvec. */
int ec_glue_embed(const void* emb, const int32_t* tok, float* x, uint32_t n_seq, uint32_t H, uint32_t vocab,
                  void* stream);
/* Embedding rows of a Q8_0 (GGUF blocks), F16 or F32 table [vocab][H]
 * (echo-core-zig/src/inference/engine.zig:30-54). */
int ec_glue_embed_fmt(int fmt, const void* emb, const int32_t* tok, float* x, uint32_t n_seq, uint32_t H,
                      uint32_t vocab, void* stream);
int ec_glue_rmsnorm_quant(const float* x, const float* w, void* act, uint32_t M, uint32_t H, void* stream);
/* x_out = x + parts[0] + ... + parts[nparts-1] (added in that order; parts is
 * [nparts][M][H], the output of ec_matvec_split), then RMSNorm + quantize of
 * x_out as ec_glue_rmsnorm_quant.  1 <= nparts <= 8; x_out must not be x. */
int ec_glue_add_rmsnorm_quant(const float* x, const float* parts, uint32_t nparts, float* x_out, const float* w,
                              void* act, uint32_t M, uint32_t H, void* stream);
int ec_glue_swiglu_quant(const float* gu, void* act, uint32_t M, uint32_t F, void* stream);
/* ec_glue_swiglu_quant over nparts (1..8) partial sums gu[nparts][M][2F], added in part order. */
int ec_glue_swiglu_quant_split(const float* gu, uint32_t nparts, void* act, uint32_t M, uint32_t F, void* stream);
/* conv_state [n_seq][kern][conv_dim] is a ring over positions: slot p % kern
 * holds the conv input of position p (all zero before position 0). */
int ec_glue_conv_gates(const float* proj, uint32_t Nin, float* conv_state, const float* conv_w, const float* a_log,
                       const float* dt_bias, float* q, float* k, float* v, float* dec, float* beta,
                       const int32_t* pos, uint32_t n_seq, uint32_t n_k, uint32_t n_v, uint32_t kern, void* stream);
int ec_glue_gated_norm_quant(const float* core, const float* proj, uint32_t Nin, uint32_t z_off, const float* norm_w,
                             void* act, uint32_t M, uint32_t n_v, void* stream);
/* The _quant ops writing `pieces` (1 or 2) pieces per element (ec_quantize_act_pieces' layout). */
int ec_glue_rmsnorm_quant_pieces(const float* x, const float* w, void* act, uint32_t M, uint32_t H, uint32_t pieces,
                                 void* stream);
int ec_glue_add_rmsnorm_quant_pieces(const float* x, const float* parts, uint32_t nparts, float* x_out,
                                     const float* w, void* act, uint32_t M, uint32_t H, uint32_t pieces,
                                     void* stream);
int ec_glue_swiglu_quant_split_pieces(const float* gu, uint32_t nparts, void* act, uint32_t M, uint32_t F,
                                      uint32_t pieces, void* stream);
int ec_glue_gated_norm_quant_pieces(const float* core, const float* proj, uint32_t Nin, uint32_t z_off,
                                    const float* norm_w, void* act, uint32_t M, uint32_t n_v, uint32_t pieces,
                                    void* stream);
int ec_glue_qk_rope_append(const float* proj, uint32_t Nin, const float* q_norm, const float* k_norm, int use_qn,
                           int use_kn, const float* inv_freq, const int32_t* pos, float* q_out, void* q_packed,
                           float* q_scales, int8_t* keys, int8_t* vals, float* kscales, float* vscales, int32_t* ctx,
                           uint32_t n_seq, uint64_t seq_stride, uint32_t max_ctx, uint32_t n_heads, uint32_t n_kv,
                           uint32_t head_dim, void* stream);
/* ec_glue_qk_rope_append with the projection given as nparts (1..8) partial
 * sums proj[nparts][n_seq][Nin] (ec_matvec_split's output), added in part order. */
int ec_glue_qk_rope_append_split(const float* proj, uint32_t nparts, uint32_t Nin, const float* q_norm,
                                 const float* k_norm, int use_qn, int use_kn, const float* inv_freq,
                                 const int32_t* pos, float* q_out, void* q_packed, float* q_scales, int8_t* keys,
                                 int8_t* vals, float* kscales, float* vscales, int32_t* ctx, uint32_t n_seq,
                                 uint64_t seq_stride, uint32_t max_ctx, uint32_t n_heads, uint32_t n_kv,
                                 uint32_t head_dim, void* stream);
/* Greedy pick (first maximum) of every active sequence (pos[s] >= 0):
 * gen[s] = next[s] = argmax, pos[s] += 1.  The _bounded form stops a
 * sequence at the cache end: when the new position would be >= max_pos (the
 * KV cache length; 0 = no limit) the sequence is instead made inactive,
 * pos[s] = -1, after its last token is written to gen.
 * ec_glue_argmax_advance keeps its original signature and has no limit
 * (max_pos = 0). */
int ec_glue_argmax_advance(const float* logits, uint32_t vocab, int32_t* gen, int32_t* next, int32_t* pos,
                           uint32_t n_seq, void* stream);
int ec_glue_argmax_advance_bounded(const float* logits, uint32_t vocab, int32_t* gen, int32_t* next, int32_t* pos,
                                   uint32_t n_seq, uint32_t max_pos, void* stream);
/* The same pick in two launches over more CUs: each row cut into `slices`
 * (1 .. 1024) ranges whose picks go to ws (ec_glue_argmax_ws_bytes(n_seq,
 * slices) bytes), then merged per sequence; identical results.  Calls sharing
 * ws must not overlap. */
size_t ec_glue_argmax_ws_bytes(uint32_t n_seq, uint32_t slices);
int ec_glue_argmax_advance_sliced(const float* logits, uint32_t vocab, int32_t* gen, int32_t* next, int32_t* pos,
                                  uint32_t n_seq, uint32_t max_pos, uint32_t slices, void* ws, void* stream);

/* ------------------------------------------------- chunked prefill glue
 * T consecutive tokens of ONE sequence at positions p0 .. p0+T-1.
 * conv_gates_chunk: as ec_glue_conv_gates for every token of the chunk (taps
 * of positions >= p0 from earlier proj rows, older ones from the ring, whose
 * slots are then overwritten with the chunk's last min(T, kern) inputs); ring
 * is the sequence's [kern][conv_dim] conv state; q, k, v, dec, beta are the
 * ec_deltanet inputs for n_seq = 1.  The _rows ops are the fp32 values of
 * ec_glue_rmsnorm_quant / ec_glue_swiglu_quant / ec_glue_gated_norm_quant
 * before quantization (quantize with ec_gemm_quantize_act for the GEMM).
 * ec_glue_qk_rope_append and ec_attn_decode[_packed] with seq_stride == 0
 * treat their n_seq slots as tokens of one sequence sharing one cache (slot s
 * at position pos[s], attending over ctx[s] positions): causal attention of a
 * chunk when ctx[s] = pos[s] + 1. */
int ec_glue_conv_gates_chunk(const float* proj, uint32_t Nin, float* ring, const float* conv_w, const float* a_log,
                             const float* dt_bias, float* q, float* k, float* v, float* dec, float* beta, uint32_t T,
                             uint32_t p0, uint32_t n_k, uint32_t n_v, uint32_t kern, void* stream);
int ec_glue_rmsnorm_rows(const float* x, const float* w, float* y, uint32_t M, uint32_t H, void* stream);
int ec_glue_swiglu_rows(const float* gu, float* y, uint32_t M, uint32_t F, void* stream);
int ec_glue_gated_norm_rows(const float* core, const float* proj, uint32_t Nin, uint32_t z_off, const float* norm_w,
                            float* y, uint32_t M, uint32_t n_v, void* stream);
/* The same three ops with their output quantized straight into the prefill
 * GEMM's Q8_0 activation layout (ec_gemm_act_bytes(EC_Q8_0, M, K) bytes, K =
 * H, F or n_v*128): byte for byte what the _rows op followed by
 * ec_gemm_quantize_act(EC_Q8_0, ...) writes, one launch instead of two.
 * rmsnorm: H % 32 == 0 and H <= 4096; swiglu: F % 32 == 0. */
int ec_glue_rmsnorm_rows_gemm_act(const float* x, const float* w, void* act, uint32_t M, uint32_t H, void* stream);
int ec_glue_swiglu_rows_gemm_act(const float* gu, void* act, uint32_t M, uint32_t F, void* stream);
int ec_glue_gated_norm_rows_gemm_act(const float* core, const float* proj, uint32_t Nin, uint32_t z_off,
                                     const float* norm_w, void* act, uint32_t M, uint32_t n_v, void* stream);

/* Plain streaming read of `bytes` (multiple of 16) with `blocks` workgroups of
 * 256 threads: the HBM-bandwidth calibration used by the benchmarks. */
int ec_stream_read(const void* src, size_t bytes, uint32_t* out, uint32_t blocks, void* stream);
/* The same read with `threads` (256/512/1024) per workgroup and `unroll`
 * (1/2/4/8) non-temporal 16-byte loads in flight per thread: the sweep that
 * finds the fastest single launch reading a buffer of a given size. */
int ec_stream_read_shape(const void* src, size_t bytes, uint32_t* out, uint32_t blocks, uint32_t threads,
                         uint32_t unroll, void* stream);

/* ----------------------------------------------------------------- random
 * Fill device memory from the portable splitmix64 stream: element i gets
 * bits of splitmix64(seed, i) (echohip/synth.py).  kind 0: uint8 bytes (low
 * byte); 1: Q8_0 GGUF weights (qs ~ U{-127..127}, d = fp16(|N(0,1)|*scale));
 * 2: fp32 N(0,1)*scale. */
int ec_fill_random(int kind, void* dst, uint64_t n, uint64_t seed, float scale, uint32_t K, void* stream);

#ifdef __cplusplus
}
#endif
#endif
