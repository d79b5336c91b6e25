/*
 * echo_engine.h — C ABI of the device-resident hybrid decoder (libechohip.so).
 *
 * The model is the reference's hybrid Qwen3.5 stack
 * (echo-core-zig/src/inference/engine.zig:360-463): n_layers blocks, block i
 * is full attention iff (i+1) % attn_interval == 0
 * (echo-core-zig/src/ports/inference.zig:135-140), otherwise a gated-delta-net
 * ("qwen_linear") block (echo-core-zig/src/kernels/qwen_linear.zig:103-271);
 * each block is followed by a SwiGLU FFN; RMSNorm before every sub-block,
 * greedy argmax at the end.  Matrices are GGUF Q8_0 or Q4_K (per tensor).
 *
 * The engine decodes a batch of up to max_batch sequences per step, each at
 * its own position (ragged).  Inputs of a step are, per sequence, a token and
 * a position (position < 0: sequence inactive this step; its state, KV cache
 * and position are untouched).  After a step the greedy next token of every
 * active sequence is in the engine's `gen` array and its position has
 * advanced by one; the next step consumes `gen` as input unless new inputs
 * are set.  A sequence that has written the last slot of its KV cache
 * (position max_ctx - 1) still gets its greedy token in `gen`, and its
 * position becomes -1 (inactive) instead of max_ctx: it stops until new
 * inputs are set.  A step runs as one captured HIP graph on the engine's stream.
 *
 * Differences from the reference, all deliberate:
 *  - activations entering a matvec are quantized per 32-element block with the
 *    reference quantizer (src/kernels/quant.cpp:18-98), plus (by default) a
 *    second int8 piece for the residual at 1/256 of the block scale, and
 *    multiplied with int8 MFMA (exact int32 block dots, fp32 scale epilogue);
 *    the prefill GEMMs use the one-piece activation;
 *  - the INT8 KV cache has one scale per (token, kv head) row, the layout its
 *    readers index (src/inference.cpp:347,387) (the reference writers store
 *    one scale per token);
 *  - an attention block attends over its own layer's cache length (the
 *    reference reads layer 0's, echo-core-zig/src/kv_cache/cache.zig:131-134,
 *    which a hybrid stack whose layer 0 is a delta-net block never appends to).
 */
#ifndef ECHO_ENGINE_H
#define ECHO_ENGINE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ec_engine ec_engine;

typedef struct {
    uint32_t vocab, hidden, ffn, n_layers;
    uint32_t n_heads, n_kv, head_dim;  /* attention blocks (head_dim 256) */
    uint32_t ssm_inner, ssm_heads;     /* delta-net value_dim and value heads (head dims 128) */
    uint32_t conv_kernel;              /* causal depthwise conv taps */
    uint32_t attn_interval;
    uint32_t max_batch, max_ctx;
    float rope_base;
} ec_engine_cfg;

/* Tensor ids for ec_engine_set_tensor.  Matrices are GGUF bytes of their
 * format (ec_engine_set_format; Q8_0 by default): rows x (K/32*34) for Q8_0,
 * rows x (K/256*144) for Q4_K; vectors are fp32.  Per-layer tensors: */
enum ec_tensor {
    EC_T_EMBED = 0,      /* [vocab x hidden] Q8_0 blocks, F16 or F32 rows (global) */
    EC_T_FINAL_NORM = 1, /* [hidden] (global) */
    EC_T_LM_HEAD = 2,    /* [vocab x hidden] (global) */
    EC_T_ATTN_NORM = 10, /* [hidden] */
    EC_T_FFN_NORM = 11,  /* [hidden] */
    EC_T_W_IN = 12,      /* delta: rows qkv(conv_dim) | z(ssm_inner) | alpha(ssm_heads) | beta(ssm_heads);
                            attention: rows q(n_heads*hd) | k(n_kv*hd) | v(n_kv*hd); K = hidden */
    EC_T_W_OUT = 13,     /* delta: [hidden x ssm_inner]; attention: [hidden x n_heads*hd] */
    EC_T_W_GATE = 14,    /* [ffn x hidden] */
    EC_T_W_UP = 15,      /* [ffn x hidden] */
    EC_T_W_DOWN = 16,    /* [hidden x ffn] */
    EC_T_CONV_W = 17,    /* delta: [conv_kernel][conv_dim], tap-major (qwen_linear.zig:197) */
    EC_T_A_LOG = 18,     /* delta: [ssm_heads] */
    EC_T_DT_BIAS = 19,   /* delta: [ssm_heads] */
    EC_T_SSM_NORM = 20,  /* delta: [128] */
    EC_T_Q_NORM = 21,    /* attention: [head_dim]; all zero = not applied (engine.zig:548-553) */
    EC_T_K_NORM = 22,    /* attention: [head_dim] */
};

int ec_engine_create(const ec_engine_cfg* cfg, ec_engine** out);
/* Storage format of a matrix, chosen per tensor as the reference's matvec_d
 * dispatch does (src/inference.cpp:526-545): EC_Q8_0 (default) or EC_Q4_K
 * (K % 256 == 0) for EC_T_W_IN, EC_T_W_OUT, EC_T_W_GATE / EC_T_W_UP (one format
 * for both: they are stored as one matrix), EC_T_W_DOWN and EC_T_LM_HEAD;
 * EC_Q8_0, EC_F16 or EC_F32 rows for EC_T_EMBED.  Reallocates the tensor (its
 * contents are undefined until set) and drops the captured step graph. */
int ec_engine_set_format(ec_engine* e, int layer, int tensor, int fmt);
int ec_engine_get_format(const ec_engine* e, int layer, int tensor);
/* int8 pieces per activation element entering the decode step's matvecs (and
 * the last prompt token's vocab projection): 2 (default) = the reference
 * quantizer's int8 plus its residual at 1/256 of the block scale
 * (ec_quantize_act_pieces; each matvec within ~2e-5 relative of the
 * reference's fp32-activation arithmetic, src/kernels/matvec.cpp:62-142), 1 =
 * the reference quantizer alone (~5e-3).  No counterpart in the reference.
 * Drops the captured step graph. */
int ec_engine_set_act_pieces(ec_engine* e, uint32_t pieces);
int ec_engine_get_act_pieces(const ec_engine* e);
/* The configuration the engine was created with. */
int ec_engine_get_config(const ec_engine* e, ec_engine_cfg* out);
void ec_engine_destroy(ec_engine* e);
/* Copy one tensor from host memory (layer ignored for global tensors). */
int ec_engine_set_tensor(ec_engine* e, int layer, int tensor, const void* host, size_t bytes);
/* Copy one tensor back to host memory in the set_tensor format (matrices as
 * GGUF bytes of their format; EC_T_W_GATE / EC_T_W_UP each return their half). */
int ec_engine_get_tensor(ec_engine* e, int layer, int tensor, void* host, size_t bytes);

/* Recurrent and cached state of one sequence after the last completed step
 * (synchronizes the engine stream), copied to host memory:
 *   EC_S_CONV     delta-net: fp32 [conv_kernel][conv_dim], a ring over
 *                 positions (slot p % conv_kernel = conv input of position p)
 *   EC_S_SSM      delta-net: fp32 [ssm_heads][128 v][128 k] (S transposed)
 *   EC_S_KEYS/VALS        attention: int8 [max_ctx][n_kv][head_dim]
 *   EC_S_KSCALES/VSCALES  attention: fp32 [max_ctx][n_kv]
 * bytes must equal the state's size. */
enum {
    EC_S_CONV = 0,
    EC_S_SSM = 1,
    EC_S_KEYS = 2,
    EC_S_VALS = 3,
    EC_S_KSCALES = 4,
    EC_S_VSCALES = 5,
};
int ec_engine_get_state(ec_engine* e, int layer, int which, uint32_t seq, void* host, size_t bytes);
/* Fill every tensor with seeded synthetic values generated on the device:
 * matrices Q8_0 with qs ~ U{-127..127} and d = fp16(|N(0,1)| * w_scale);
 * norms 1 + 0.1*N(0,1); conv taps 0.5*N(0,1); A_log = ln U[1,16]; dt_bias 0.1*N(0,1). */
int ec_engine_init_random(ec_engine* e, uint64_t seed, float w_scale);
/* Zero recurrent state, conv state and KV caches; all positions inactive. */
int ec_engine_reset(ec_engine* e);
/* Set this step's inputs for n <= max_batch sequences (host arrays). */
int ec_engine_set_inputs(ec_engine* e, const int32_t* tok, const int32_t* pos, uint32_t n);
/* Chunked prefill of one sequence: feed n tokens at positions pos0 ..
 * pos0+n-1 (the sequence's next position; pos0 + n <= max_ctx) in chunks of up
 * to 512 tokens, each block computed for the whole chunk (int8-MFMA GEMMs,
 * the delta rule over the chunk's tokens, causal attention of every token over
 * the sequence's cache).  Leaves the sequence as n decode steps would
 * (conv/recurrent state, KV cache, position pos0 + n, greedy next token in
 * `gen`, the last token's logits); other sequences are untouched.  Synchronous. */
int ec_engine_prefill(ec_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n, int32_t pos0);
/* ec_engine_prefill of n_seqs distinct sequences (seqs[i], tokens[i][0 ..
 * lens[i]), positions from pos0[i]); two sequences' chunks at a time share
 * each row op and GEMM (one launch over both chunks' rows), two such passes
 * run concurrently on two streams, each sequence's result bit for bit that of
 * ec_engine_prefill.  Synchronous. */
int ec_engine_prefill_batch(ec_engine* e, uint32_t n_seqs, const uint32_t* seqs, const int32_t* const* tokens,
                            const uint32_t* lens, const int32_t* pos0);
/* Run one decode step (graph-captured after the first call when use_graph). */
int ec_engine_step(ec_engine* e, int use_graph);
int ec_engine_sync(ec_engine* e);
/* Device -> host copies (synchronous). */
int ec_engine_get_tokens(ec_engine* e, int32_t* gen, int32_t* pos);
int ec_engine_get_logits(ec_engine* e, float* host, uint32_t seq);
void* ec_engine_stream(ec_engine* e);
/* HBM bytes of weights one decode step reads (tiled Q8_0 matrices + vectors). */
size_t ec_engine_weight_bytes(const ec_engine* e);
/* Decode-step matvec timing: the step's Q8_0 matvec launches alone (same
 * shapes, buffers and order as in the step) are captured into a separate HIP
 * graph, replayed `reps` times between two HIP events on the engine stream.
 * Reports the launches per step, their algorithmic bytes per step and GPU
 * microseconds per step.  Matvecs read weights and activations and write
 * scratch outputs only: the recurrent state, KV cache and positions are not
 * touched, so decoding can continue afterwards (the next step recomputes the
 * scratch). */
int ec_engine_profile_matvecs(ec_engine* e, uint32_t reps, uint32_t* launches, double* bytes_per_step,
                              double* us_per_step);

/* ------------------------------------------------------------ step tracing
 * For checking the decode step one operation at a time: the step's launches
 * (the same kernels, buffers and order as ec_engine_step) run eagerly, and
 * around every launch the engine stream is synchronized and cb is called
 * twice, before (phase 0) and after (phase 1) the launch, so the callback
 * can read the operation's inputs and outputs (ec_engine_buffer,
 * ec_engine_get_state).  Not for production use: every launch waits. */
enum {
    EC_OP_EMBED = 0,       /* tok -> x */
    EC_OP_NORM = 1,        /* x_in (+ nparts partial sums in PARTS) -> x_out, ACT_H; RMSNorm + quantize */
    EC_OP_MV_IN = 2,       /* ACT_H -> PROJ [nparts][B][Nin] (delta: q|k|v|z|alpha|beta, attention: q|k|v) */
    EC_OP_DELTA_STEP = 3,  /* PROJ, conv and recurrent state -> state, ACT_V */
    EC_OP_MV_OUT = 4,      /* ACT_V or ACT_Q -> PARTS [nparts][B][H] */
    EC_OP_ROPE_APPEND = 5, /* PROJ -> KV row at pos, Q_PACKED + Q_SCALES (or QBUF), CTX */
    EC_OP_ATTN = 6,        /* Q_PACKED (or QBUF), KV cache, CTX -> ATTN_OUT (and ACT_Q when packed) */
    EC_OP_QUANT_ACT = 7,   /* fp32 rows (buffer x_in) -> activation (buffer x_out): ATTN_OUT -> ACT_Q (fp32
                              attention), and the inputs of Q4_K matrices (HN, CORE, ATTN_OUT, FF -> ACT4_*) */
    EC_OP_MV_GU = 8,       /* ACT_H -> GU [nparts][B][2F] (gate rows, then up rows) */
    EC_OP_SWIGLU = 9,      /* GU -> ACT_F, or fp32 FF rows (x_out says which) */
    EC_OP_MV_DOWN = 10,    /* ACT_F -> PARTS [nparts][B][H] */
    EC_OP_LM_HEAD = 11,    /* ACT_H -> LOGITS */
    EC_OP_ARGMAX = 12,     /* LOGITS, POS -> GEN, TOK, POS */
    EC_OP_NORM_ROWS = 13,  /* x_in -> HN: the fp32 RMSNorm rows a Q4_K consumer quantizes */
    /* chunked prefill (ec_engine_prefill_traced), rows = the chunk's T tokens,
       buffers EC_B_PF_*: */
    EC_OP_PF_EMBED = 20,      /* PF_TOK -> PF_X */
    EC_OP_PF_NORM = 21,       /* PF_X -> PF_N: RMSNorm rows (attention / ffn norm, then the final norm) */
    EC_OP_PF_GEMM_IN = 22,    /* PF_N -> PF_PROJ [T][Nin]: activation quantized per row, int8-MFMA GEMM */
    EC_OP_PF_CONV = 23,       /* PF_PROJ, conv ring -> PF_Q, PF_K, PF_V, PF_DEC, PF_BETA, ring */
    EC_OP_PF_DELTA = 24,      /* PF_Q .. PF_BETA, recurrent state -> PF_CORE, state */
    EC_OP_PF_GATED_NORM = 25, /* PF_CORE, PF_PROJ (z) -> PF_N */
    EC_OP_PF_GEMM_OUT = 26,   /* PF_N (delta) or PF_ATTN -> PF_X += */
    EC_OP_PF_ROPE_APPEND = 27,/* PF_PROJ -> PF_N (q rows), KV rows of the chunk */
    EC_OP_PF_ATTN = 28,       /* PF_N (q rows), KV cache -> PF_ATTN */
    EC_OP_PF_GEMM_GU = 29,    /* PF_N -> PF_GU [T][2F] */
    EC_OP_PF_SWIGLU = 30,     /* PF_GU -> PF_N [T][F] */
    EC_OP_PF_GEMM_DOWN = 31,  /* PF_N -> PF_X += */
    EC_OP_PF_HEAD = 32,       /* last row of PF_X -> LOGITS row of the sequence (final RMSNorm, quantize, head) */
};
typedef struct {
    int op, layer;   /* layer -1: embedding, final norm, head, argmax */
    int phase;       /* 0: before the launch, 1: after it completed */
    int nparts;      /* partial sums the op writes (MV_*) or reads (NORM, DELTA_STEP, ROPE_APPEND, SWIGLU) */
    int x_in, x_out; /* EMBED / NORM / NORM_ROWS: the residual buffers (EC_B_X / EC_B_X2) read and written;
                        MV_*: x_in = the activation buffer read; QUANT_ACT: source and destination buffers;
                        DELTA_STEP / SWIGLU / ATTN: x_out = the output buffer (ACT_V or CORE, ACT_F or FF,
                        ACT_Q or -1); else -1 */
} ec_trace_event;
typedef void (*ec_trace_fn)(void* user, const ec_trace_event* ev);
int ec_engine_step_traced(ec_engine* e, ec_trace_fn cb, void* user);
/* ec_engine_prefill of one sequence with cb called around every launch (one
 * lane, so chunks run in order); layer -1 for the embedding and the head.
 * The chunk buffers are EC_B_PF_* (rows = up to 512 tokens). */
int ec_engine_prefill_traced(ec_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n, int32_t pos0,
                             ec_trace_fn cb, void* user);

/* Device address and size of one of the engine's step buffers (activation
 * buffers in the ec_quantize_act layout, M = max_batch). */
enum {
    EC_B_X = 0, EC_B_X2 = 1, EC_B_PARTS = 2, EC_B_PROJ = 3, EC_B_GU = 4, EC_B_ACT_H = 5, EC_B_ACT_V = 6,
    EC_B_ACT_F = 7, EC_B_ACT_Q = 8, EC_B_ATTN_OUT = 9, EC_B_Q_PACKED = 10, EC_B_Q_SCALES = 11, EC_B_QBUF = 12,
    EC_B_LOGITS = 13, EC_B_TOK = 14, EC_B_POS = 15, EC_B_GEN = 16, EC_B_CTX = 17, EC_B_INV_FREQ = 18,
    /* inputs of Q4_K matrices (present once a matrix is Q4_K): fp32 rows and their Q4_K activations */
    EC_B_HN = 19, EC_B_CORE = 20, EC_B_FF = 21, EC_B_ACT4_H = 22, EC_B_ACT4_V = 23, EC_B_ACT4_Q = 24,
    EC_B_ACT4_F = 25,
    /* chunked prefill, lane 0 (allocated by the first prefill): fp32 rows [512][...] */
    EC_B_PF_X = 30, EC_B_PF_N = 31, EC_B_PF_PROJ = 32, EC_B_PF_Q = 33, EC_B_PF_K = 34, EC_B_PF_V = 35,
    EC_B_PF_DEC = 36, EC_B_PF_BETA = 37, EC_B_PF_CORE = 38, EC_B_PF_GU = 39, EC_B_PF_ATTN = 40, EC_B_PF_TOK = 41,
    EC_B_PF_ACT1 = 42, /* the last token's head activation (Q8_0 or Q4_K layout, M = 1) */
    EC_B_PF_ACT = 43,  /* the chunk's GEMM activation (ec_gemm_quantize_act layout of the GEMM's format and K) */
};
int ec_engine_buffer(ec_engine* e, int which, void** dev, size_t* bytes);

#ifdef __cplusplus
}
#endif
#endif
