/*
 * oracle.h — CPU restatement of echo-core's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it; the product library (libechohip.so) never links, loads or calls it.
 *
 * Every function cites the reference file:line whose algorithm it restates
 * (paths relative to the echo-core source tree).  Functions marked "design"
 * restate a step this build adds (activation quantization for integer block
 * dots); they are built from the reference quantizer and pinned by the
 * tests named in their comment.
 *
 * Pinning (tests/test_oracle_*.py):
 *   fp16 codec            exhaustive over all 65536 halves vs numpy float16
 *   quantizer             reference known answers + golden vectors from the
 *                         compiled reference (oracle/_ref)
 *   q8_0 / q4_K dots      reference known answers, golden vectors, fp64 brute
 *                         force, single-nibble layout probes
 *   int8 attention        closed forms (equal keys -> mean of V, one dominant
 *                         key -> that V row, GQA modulo mapping), fp64 brute force
 *   delta-net             closed forms (one step from S0=0, beta=0 pure decay,
 *                         orthonormal-key retrieval, column permutation), fp64
 *                         brute force
 *   decoder glue          fp64 brute force per op; RoPE rotation norm invariance
 *   delta-net gates and   closed forms (softplus(0) = ln 2 gives decay
 *   gated RMSNorm         2^-exp(A_log); softplus(x > 20) = x; sigmoid(0) = 1/2;
 *                         z = 0 gives 0; a constant core gives w*c/sqrt(c^2+eps)*SiLU(z))
 *   blocks / decoder      closed forms with unit-row Q8_0 projections (delta-net
 *                         first token S = k (x) beta v, state decay, zero z; attention
 *                         at position 0 returns V of kv head h % n_kv; FFN
 *                         silu(gate)*up); oc_decoder_token equals the composition
 *                         of the blocks bit for bit (tests/test_oracle_blocks.py)
 */
#ifndef ECHO_ORACLE_H
#define ECHO_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (include/types.h:13-19: F16C decode, RNE encode) ---- */
float    oc_fp16_to_fp32(uint16_t h);
uint16_t oc_fp32_to_fp16(float f);

/* ---- portable RNG: splitmix64 stream element i (state seed, i+1 steps) ---- */
uint64_t oc_splitmix64_at(uint64_t seed, uint64_t i);

/* ---- quantizer (src/kernels/quant.cpp:18-98) ----
 * Elements in whole 8-chunks: q = sat8(rne(x * (1/scale)));
 * remaining tail: q = clamp(round_half_away(x / scale), -127, 127). */
void oc_quantize_per_token_symmetric(const float* input, int8_t* output, float* scales,
                                     uint32_t num_tokens, uint32_t num_elements);

/* ---- int8 score kernel (src/kernels/quant.cpp:100-144), scalar order ---- */
void oc_fused_dequant_dot_int8(const float* query, const int8_t* key_cache, const float* scales,
                               float* scores, uint32_t dim, uint32_t seq_len);

/* ---- row dots (src/kernels/quant.cpp:150-194, :210-304), fp64 accumulate ---- */
double oc_dot_q8_0_f64(const uint8_t* blocks, uint32_t n_blocks, const float* x);
double oc_dot_q4_K_f64(const uint8_t* blocks, uint32_t n_blocks, const float* x);

/* ---- matvec, reference summation order (src/kernels/matvec.cpp:62-87, :92-142) ----
 * y[m] += sum over row m.  blocks are GGUF bytes (34 B / 144 B blocks). */
void oc_matvec_q8_0(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K);
void oc_matvec_q4_K(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K);

/* ---- Q4_K scale/min unpack (src/kernels/quant.cpp:222-242) ---- */
void oc_q4k_scale_min(const uint8_t* scales12, int j, uint8_t* sc, uint8_t* m);
/* Position of element i (0..31) of sub-block s (0..7) inside a 256-weight
 * super-block under the reference nibble layout (src/kernels/quant.cpp:202-207,
 * :254-299): sub-block s owns qs bytes [16s, 16s+16); i<16 -> low nibble of
 * byte 16s+i, i>=16 -> high nibble of byte 16s+i-16. */
uint32_t oc_q4k_pos(uint32_t s, uint32_t i);

/* ---- activation quantization (design; built on the reference quantizer) ----
 * Q8_0 grouping: blocks of 32 consecutive elements.
 * Q4_K grouping: the 32 positions of each Q4_K sub-block (oc_q4k_pos), so
 *   every int8 block meets exactly one 6-bit scale/min pair.
 * xq is stored in block order (block-major, 32 per block); xd = scale per
 * block; xsum = sum of the block's int8 values (Q4_K min term). */
void oc_quantize_act_q8_0(const float* x, int8_t* xq, float* xd, uint32_t K);
void oc_quantize_act_q4_K(const float* x, int8_t* xq, float* xd, int32_t* xsum, uint32_t K);
/* Two-piece Q8_0 activation (design): q0 = the reference quantizer per
 * 32-block with scale s; q1 = sat8(rne(fma(-q0, s, x) * ((1/s)*256))) with
 * scale s/256.  x ~ q0*s + q1*s/256; x_deq = q0*s + q1*(s/256). */
void oc_quantize_act2_q8_0(const float* x, int8_t* xq0, int8_t* xq1, float* xd, uint32_t K);
void oc_dequant_act2_q8_0(const int8_t* xq0, const int8_t* xq1, const float* xd, float* x_deq, uint32_t K);
void oc_quantize_act2_q4_K(const float* x, int8_t* xq0, int8_t* xq1, float* xd, uint32_t K);
void oc_dequant_act2_q4_K(const int8_t* xq0, const int8_t* xq1, const float* xd, float* x_deq, uint32_t K);
/* Dequantize back to natural order (x_deq[k] = xq*xd) for the reference matvec. */
void oc_dequant_act_q8_0(const int8_t* xq, const float* xd, float* x_deq, uint32_t K);
void oc_dequant_act_q4_K(const int8_t* xq, const float* xd, float* x_deq, uint32_t K);

/* ---- exact integer block dots (closed form, the bit-exact contract) ----
 * Q8_0: out[m*(K/32)+b]   = sum_j qs[m][b][j] * xq[b*32+j]
 * Q4_K: out[m*(K/32)+8b+s]= sum_i q(m,b,s,i) * xq[(8b+s)*32+i]   (xq in Q4_K grouping) */
void oc_block_dots_q8_0(const void* blocks, const int8_t* xq, int32_t* out, uint32_t M, uint32_t K);
void oc_block_dots_q4_K(const void* blocks, const int8_t* xq, int32_t* out, uint32_t M, uint32_t K);

/* ---- KV append per (token, kv_head) (src/kv_cache.cpp:89-113 with the
 * reader's scale indexing pos*n_kv+kv_head, src/inference.cpp:347,387) ---- */
void oc_kv_append(const float* k, const float* v, int8_t* keys, int8_t* vals,
                  float* kscales, float* vscales, uint32_t pos, uint32_t n_kv, uint32_t head_dim);

/* ---- INT8 decode attention (echo-core-zig/src/inference/engine.zig:563-616,
 * math.softmax core/math.zig:39-52): kv = h % n_kv, score scaled after dot. ---- */
void oc_attn_decode_int8(const float* q, const int8_t* keys, const int8_t* vals,
                         const float* kscales, const float* vscales, float* out,
                         uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t ctx);

/* ---- gated delta-net recurrence core (echo-core-zig/src/kernels/qwen_linear.zig:207-250)
 * One token.  state: [n_v][d_k][d_v] row-major S[k*d_v+v] per head (reference layout).
 * q, k: [n_k][d_k] (already L2-normalised), v: [n_v][d_v]; decay, beta: [n_v]
 * (beta already through the sigmoid).  q head for v-head h is h / (n_v/n_k).
 * out: [n_v][d_v] = S^T (q * 1/sqrt(d_k)). */
void oc_deltanet_step(float* state, const float* q, const float* k, const float* v,
                      const float* decay, const float* beta, float* out,
                      uint32_t n_v, uint32_t n_k, uint32_t d_k, uint32_t d_v);

/* ---- decoder glue ---- */
/* RMSNorm (engine.zig:783-792): out = x * (1/sqrt(mean(x^2)+1e-6)) * w */
void oc_rmsnorm(const float* x, const float* w, float* out, uint32_t n);
/* per-head RMSNorm (engine.zig:507-518) */
void oc_head_rmsnorm(float* x, const float* w, uint32_t n_heads, uint32_t head_dim);
/* RoPE, adjacent pairs, full head_dim (engine.zig:466-504).  inv_freq[i/2] =
 * 1/pow(10000, i/head_dim) supplied by the caller (oc_rope_inv_freq). */
void oc_rope_inv_freq(float* inv_freq, uint32_t head_dim, float base);
void oc_rope(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos, const float* inv_freq);
/* SiLU (core/math.zig:35-37) */
float oc_silu(float x);
/* softplus with x>20 -> x (qwen_linear.zig:71-74) */
float oc_softplus(float x);
/* L2 normalise heads with 1/sqrt(sum+1e-6) (qwen_linear.zig:87-101) */
void oc_l2norm_heads(float* x, uint32_t n_heads, uint32_t head_dim);
/* causal depthwise conv step (qwen_linear.zig:182-201): shift conv_state
 * [kernel][C] (newest at slot 0), insert x, out[c] = silu(sum_t st[t][c]*w[(kernel-1-t)*C+c]) */
void oc_conv_step(float* conv_state, const float* x, const float* w, float* out,
                  uint32_t C, uint32_t kernel);

/* ---- full hybrid decoder (engine.zig:360-463, qwen_linear.zig:103-271) ----
 * Small, self-contained restatement used as the decoder checker and as the
 * CPU baseline.  Weights are GGUF Q8_0 byte blocks; norms and small vectors
 * are fp32.  quant_act 1 inserts the one-piece int8 activation quantization
 * before every matvec, 2 the two-piece one (oc_quantize_act2_q8_0 /
 * oc_quantize_act2_q4_K, what the GPU decode step computes by default),
 * 0 keeps fp32 activations (reference semantics). */
typedef struct {
    uint32_t hidden, ffn, n_layers, vocab;
    uint32_t n_heads, n_kv, head_dim;          /* full-attention layers */
    uint32_t ssm_inner, ssm_heads, conv_kernel; /* delta-net layers: value_dim, n_v heads */
    uint32_t attn_interval;                    /* layer i is attention iff (i+1)%interval==0 */
    uint32_t max_ctx;
    float rope_base;
} oc_model_cfg;

typedef struct {
    /* per layer, indexed by layer */
    const uint8_t** w_qkv;   /* delta: [conv_dim x hidden]; attn: [(q+2kv) x hidden] (q|k|v rows) */
    const uint8_t** w_z;     /* delta: [ssm_inner x hidden] */
    const uint8_t** w_ab;    /* delta: [2*ssm_heads x hidden] (alpha rows then beta rows) */
    const uint8_t** w_out;   /* delta: [hidden x ssm_inner]; attn o: [hidden x q_dim] */
    const uint8_t** w_gate;  /* [ffn x hidden] */
    const uint8_t** w_up;    /* [ffn x hidden] */
    const uint8_t** w_down;  /* [hidden x ffn] */
    const float** attn_norm; /* [hidden] */
    const float** ffn_norm;  /* [hidden] */
    const float** conv_w;    /* delta: [kernel][conv_dim] tap-major (qwen_linear.zig:197) */
    const float** a_log;     /* delta: [ssm_heads] */
    const float** dt_bias;   /* delta: [ssm_heads] */
    const float** ssm_norm;  /* delta: [head_v_dim] */
    const float** q_norm;    /* attn: [head_dim] */
    const float** k_norm;    /* attn: [head_dim] */
    const uint8_t* embed;    /* [vocab x hidden] Q8_0 (or per fmt) */
    const float* final_norm; /* [hidden] */
    const uint8_t* lm_head;  /* [vocab x hidden] Q8_0 (or per fmt) */
    /* Storage formats, chosen per tensor as src/inference.cpp:526-545
     * dispatches them: NULL = every matrix and the embedding Q8_0; else
     * [n_layers][4] (w_qkv|w_z|w_ab as one fused matrix, w_out, w_gate|w_up,
     * w_down) in {OC_Q8_0, OC_Q4_K}, then lm_head, then the embedding in
     * {OC_Q8_0, OC_F16, OC_F32}. */
    const int32_t* fmt;
} oc_model_w;

enum { OC_F32 = 0, OC_F16 = 1, OC_Q8_0 = 6, OC_Q4_K = 10 };

typedef struct {
    /* per layer pointers; NULL for layers of the other type */
    float** conv_state;  /* [kernel][conv_dim] */
    float** ssm_state;   /* [ssm_heads][d_k][d_v] */
    int8_t** keys;       /* [max_ctx][n_kv][head_dim] */
    int8_t** vals;
    float** kscales;     /* [max_ctx][n_kv] */
    float** vscales;
    uint32_t pos;        /* tokens already processed */
} oc_seq_state;

/* Q8_0 embedding row (engine.zig:41-50). */
void oc_embed_row_q8_0(const uint8_t* embed, uint32_t H, uint32_t token, float* x);
/* Embedding row of a table in format fmt (OC_Q8_0, OC_F16 or OC_F32 rows). */
void oc_embed_row(int fmt, const void* embed, uint32_t H, uint32_t token, float* x);
/* Delta-net gates (qwen_linear.zig:215-219) per value head:
 * beta = sigmoid(beta_logit), decay = exp(-exp(a_log) * softplus(alpha + dt_bias)). */
void oc_deltanet_gates(const float* alpha, const float* beta_logit, const float* a_log, const float* dt_bias,
                       float* decay, float* beta, uint32_t n_v);
/* Gated RMSNorm (qwen_linear.zig:244-257), in place on core [n_v][d_v]:
 * core * (1/sqrt(mean(core^2) + 1e-6)) * w * silu(z). */
void oc_gated_rmsnorm(float* core, const float* z, const float* w, uint32_t n_v, uint32_t d_v);
/* y = W x (y zeroed), x first quantized per 32-block when quant_act != 0. */
void oc_matvec_act_q8_0(const void* W, const float* x, float* y, uint32_t M, uint32_t K, int quant_act);
/* The same for a matrix of format fmt (OC_Q8_0 or OC_Q4_K; a Q4_K input is
 * quantized per 32-element sub-block, oc_quantize_act_q4_K; quant_act 2 in
 * two pieces, oc_quantize_act2_q4_K). */
void oc_matvec_act(int fmt, const void* W, const float* x, float* y, uint32_t M, uint32_t K, int quant_act);
/* qwen_linear.forward of block l (qwen_linear.zig:103-271): in = the block's
 * normed input [hidden], out = its output [hidden] (before the residual). */
void oc_deltanet_block(const oc_model_cfg* c, const oc_model_w* w, uint32_t l, float* conv_state, float* ssm_state,
                       const float* in, float* out, int quant_act);
/* Attention block l at position pos (engine.zig:520-621), appending to the
 * layer's cache before attending over pos+1 positions. */
void oc_attention_block(const oc_model_cfg* c, const oc_model_w* w, uint32_t l, int8_t* keys, int8_t* vals,
                        float* kscales, float* vscales, uint32_t pos, const float* in, float* out, int quant_act);
/* out = silu(gate) * up elementwise (engine.zig:769-772); out may alias gate. */
void oc_swiglu(const float* gate, const float* up, float* out, uint32_t n);
/* SwiGLU FFN of block l (engine.zig:748-781). */
void oc_ffn_block(const oc_model_cfg* c, const oc_model_w* w, uint32_t l, const float* in, float* out,
                  int quant_act);
/* One token of one sequence: fills logits [vocab]; advances st->pos. */
void oc_decoder_token(const oc_model_cfg* cfg, const oc_model_w* w, oc_seq_state* st,
                      uint32_t token, float* logits, int quant_act);
uint32_t oc_argmax(const float* x, uint32_t n);

#ifdef __cplusplus
}
#endif
#endif
