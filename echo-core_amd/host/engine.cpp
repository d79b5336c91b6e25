// engine.cpp — device-resident hybrid decoder behind the C ABI of echo_engine.h.
//
// Host control only: every operation is a call into libechohip's C ABI
// (echo_hip.h), launched on the engine's stream; a decode step is captured
// once into a HIP graph and replayed.  Layer structure and op order follow
// echo-core-zig/src/inference/engine.zig:397-463 (layerForward), the attention
// block :520-621 and qwen_linear.forward (kernels/qwen_linear.zig:103-271).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <utility>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "echo_engine.h"
#include "echo_hip.h"

namespace {

#define EC_HIP(call)                                                             \
    do {                                                                         \
        hipError_t _e = (call);                                                  \
        if (_e != hipSuccess) return ec_set_hip_error_host(_e, #call);           \
    } while (0)
#define EC_TRY(call)                  \
    do {                                \
        int _rc = (call);               \
        if (_rc != EC_OK) return _rc;   \
    } while (0)

extern "C" int ec_set_error(int code, const char* msg);
extern "C" int ec_set_hip_error(hipError_t e, const char* where);
int ec_set_hip_error_host(hipError_t e, const char* where) { return ec_set_hip_error(e, where); }

// splitmix64 / Box-Muller, identical to echohip/synth.py.
uint64_t sm64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
double u01(uint64_t z) { return (double)(z >> 40) * (1.0 / 16777216.0); }
double normal_at(uint64_t seed, uint64_t i) {
    double a = 1.0 - u01(sm64(seed, 2 * i)), b = u01(sm64(seed, 2 * i + 1));
    return std::sqrt(-2.0 * std::log(a)) * std::cos(6.283185307179586 * b);
}

struct Mat {
    void* tiled = nullptr;
    uint32_t N = 0, K = 0;
    int fmt = EC_Q8_0;  // EC_Q8_0 or EC_Q4_K (src/inference.cpp:526-545 dispatches per tensor)
};

struct Layer {
    bool attn = false;
    Mat w_in, w_out, w_gu, w_down;
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    float* conv_w = nullptr;
    float* a_log = nullptr;
    float* dt_bias = nullptr;
    float* ssm_norm = nullptr;
    float* conv_state = nullptr;
    float* ssm_state = nullptr;
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    int use_qn = 0, use_kn = 0;
    int8_t* keys = nullptr;
    int8_t* vals = nullptr;
    float* ks = nullptr;
    float* vs = nullptr;
};

}  // namespace

struct ec_engine {
    ec_engine_cfg c{};
    hipStream_t st = nullptr;
    std::vector<Layer> L;
    void* embed = nullptr;
    int embed_fmt = EC_Q8_0;  // EC_Q8_0 (GGUF blocks), EC_F16 or EC_F32 rows
    float* final_norm = nullptr;
    Mat lm_head;
    uint32_t B = 0, H = 0, F = 0, q_dim = 0, kv_dim = 0, value_dim = 0, key_dim = 0, conv_dim = 0, n_v = 0, n_k = 0;
    uint32_t nin_delta = 0, nin_attn = 0, nin_max = 0;
    uint64_t seq_stride = 0;  // bytes between sequences' K (V) caches: ctx_stride positions
    uint32_t ctx_stride = 0;  // cache positions per sequence (>= max_ctx)
    float *x = nullptr, *proj = nullptr, *gu = nullptr, *core = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    // decode residual stream: x and x2 alternate (each fused residual add
    // writes the other one); parts holds a split-K projection's partial sums
    float *x2 = nullptr, *parts = nullptr;
    float *dec = nullptr, *beta = nullptr, *qbuf = nullptr, *attn_out = nullptr, *logits = nullptr;
    float* inv_freq = nullptr;
    void *act_h = nullptr, *act_v = nullptr, *act_f = nullptr, *act_q = nullptr, *attn_ws = nullptr;
    void* am_ws = nullptr;  // per-slice picks of the greedy argmax
    void* q_packed = nullptr;
    float* q_scales = nullptr;
    // inputs of Q4_K matrices (allocated with the first one): fp32 rows of the
    // producing op and their Q4_K-grouped activation
    bool q4 = false;
    float *hn = nullptr, *core_f = nullptr, *ff = nullptr;
    void *act4_h = nullptr, *act4_v = nullptr, *act4_q = nullptr, *act4_f = nullptr;
    bool packed_attn = false;  // int8-MFMA attention with q packed by the rope kernel
    // int8 pieces per activation element of the decode step's matvecs (1: the
    // reference quantizer alone; 2: plus the residual at scale/256, within
    // ~2e-5 of the fp32-activation matvec); buffers are sized for 2
    uint32_t P = 2;
    int32_t *tok = nullptr, *pos = nullptr, *gen = nullptr, *ctx = nullptr;
    // pinned staging for ec_engine_set_inputs: a ring of slots (tok[16],
    // pos[16]), each reused only after the event recorded behind its copies
    // has completed, so the host never overwrites inputs a queued copy has
    // not read yet
    static constexpr uint32_t kIoSlots = 64;
    int32_t* h_io = nullptr;
    hipEvent_t io_ev[kIoSlots] = {};
    bool io_pending[kIoSlots] = {};
    uint32_t io_next = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<void*> allocs;
    size_t weight_bytes = 0;
    // profiling hooks (eager step only)
    // matvec-only recording (profiling): skip every other launch, collect bytes
    bool mv_only = false;
    std::vector<double>* mv_bytes = nullptr;
    // step tracing (ec_engine_step_traced): called around every launch
    ec_trace_fn trace_cb = nullptr;
    void* trace_user = nullptr;
    // chunked prefill: lanes of scratch rows (a pass of up to kPrefillGroup
    // sequences' chunks of kPrefillChunk tokens each, ~170 MB per sequence at
    // 4B shapes) with their own stream, allocated on first use; lane 0 runs
    // on st.  A lane's pass runs its sequences' chunks through the row ops and
    // GEMMs together; several lanes' passes run concurrently.
    static constexpr uint32_t kPrefillChunk = 512, kPrefillAttnSlots = 128, kPrefillLanes = 4, kPrefillGroup = 4;
    struct PrefillLane {
        bool ready = false;
        uint32_t rows = 0;  // row capacity: group x kPrefillChunk
        hipStream_t st = nullptr;
        float *x = nullptr, *n = nullptr, *proj = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
        float *dec = nullptr, *beta = nullptr, *core = nullptr, *gu = nullptr, *attn = nullptr;
        void *act = nullptr, *ws = nullptr, *act1 = nullptr;  // act1: one row, for the last token's logits
        size_t act_bytes = 0;
        void* dnws = nullptr;  // chunked delta-net workspace
        void* aws = nullptr;   // segment partials of the chunk attention
        int32_t *tok = nullptr, *pos = nullptr, *ctx = nullptr;
        std::vector<int32_t> h_pos;
    };
    PrefillLane pf[kPrefillLanes];
};

namespace {

int dalloc(ec_engine* e, void** p, size_t bytes) {
    EC_HIP(hipMalloc(p, bytes ? bytes : 16));
    EC_HIP(hipMemsetAsync(*p, 0, bytes ? bytes : 16, e->st));
    e->allocs.push_back(*p);
    return EC_OK;
}
template <class T>
int dalloc(ec_engine* e, T** p, size_t count) {
    return dalloc(e, (void**)p, count * sizeof(T));
}

int alloc_mat(ec_engine* e, Mat& m, uint32_t N, uint32_t K) {
    m.N = N;
    m.K = K;
    return dalloc(e, &m.tiled, ec_tiled_bytes(m.fmt, N, K));
}

bool is_attn(const ec_engine_cfg& c, uint32_t l) { return c.attn_interval && ((l + 1) % c.attn_interval) == 0; }

size_t gguf_bytes(int fmt, uint32_t N, uint32_t K) {
    return fmt == EC_Q4_K ? (size_t)N * (K / 256) * 144 : (size_t)N * (K / 32) * 34;
}
size_t gguf_bytes(const Mat& m, uint32_t N) { return gguf_bytes(m.fmt, N, m.K); }
size_t embed_bytes(const ec_engine* e) {
    const size_t n = (size_t)e->c.vocab * e->H;
    return e->embed_fmt == EC_F16 ? 2 * n : (e->embed_fmt == EC_F32 ? 4 * n : gguf_bytes(EC_Q8_0, e->c.vocab, e->H));
}

// Upload GGUF bytes (host) of rows [row0, row0+N) of matrix m's logical rows
// and repack them into the tiled layout at that tile offset (row0 % 16 == 0).
int upload_rows(ec_engine* e, Mat& m, uint32_t row0, const void* host, uint32_t N) {
    if (row0 % 16 || row0 + N > m.N) return ec_set_error(EC_ERR_ARG, "engine: bad row range");
    void* tmp = nullptr;
    EC_HIP(hipMalloc(&tmp, gguf_bytes(m, N)));
    EC_HIP(hipMemcpyAsync(tmp, host, gguf_bytes(m, N), hipMemcpyHostToDevice, e->st));
    uint8_t* dst = (uint8_t*)m.tiled + ec_tiled_bytes(m.fmt, row0, m.K);
    int rc = ec_repack(m.fmt, tmp, dst, N, m.K, e->st);
    EC_HIP(hipStreamSynchronize(e->st));
    EC_HIP(hipFree(tmp));
    return rc;
}

int random_rows(ec_engine* e, Mat& m, uint32_t row0, uint32_t N, uint64_t seed, float scale, void* tmp) {
    if (m.fmt != EC_Q8_0) return ec_set_error(EC_ERR_UNSUPPORTED, "ec_engine_init_random: Q8_0 matrices only");
    EC_TRY(ec_fill_random(1, tmp, (uint64_t)N * (m.K / 32), seed, scale, m.K, e->st));
    uint8_t* dst = (uint8_t*)m.tiled + ec_tiled_bytes(EC_Q8_0, row0, m.K);
    return ec_repack(EC_Q8_0, tmp, dst, N, m.K, e->st);
}

// Host <-> device copies on the engine stream, complete on return.  The
// engine's buffers are zeroed and written by work queued on its non-blocking
// stream, which a copy on the null stream would not wait for.
int h2d(ec_engine* e, void* dst, const void* src, size_t bytes) {
    EC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, e->st));
    EC_HIP(hipStreamSynchronize(e->st));
    return EC_OK;
}
int d2h(ec_engine* e, void* dst, const void* src, size_t bytes) {
    EC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, e->st));
    EC_HIP(hipStreamSynchronize(e->st));
    return EC_OK;
}

int upload_vec(ec_engine* e, float* dst, const std::vector<float>& v) {
    return h2d(e, dst, v.data(), v.size() * sizeof(float));
}

std::vector<float> gen_vec(uint64_t seed, size_t n, double mean, double std) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (float)(mean + std * normal_at(seed, i));
    return v;
}

// Activation bytes of one matvec input (int8 + fp32 block scales; Q4_K also
// fp32 per-block sums).
double act_alg_bytes(const ec_engine* e, const Mat& m) {
    return (double)e->B * (e->P * m.K + m.K / 32 * 4 * (m.fmt == EC_Q4_K ? 2 : 1));
}

// One matvec launch; in profiling mode also its algorithmic bytes (weights,
// activation bytes + scales, outputs written, and read too when accumulating).
int mv(ec_engine* e, const Mat& m, const void* act, float* y, uint32_t ldy, int acc) {
    if (e->mv_bytes)
        e->mv_bytes->push_back((double)gguf_bytes(m, m.N) + act_alg_bytes(e, m) +
                               (double)e->B * m.N * 4 * (acc ? 2 : 1));
    return ec_matvec_pieces(m.fmt, e->P, m.tiled, act, y, e->B, m.N, m.K, ldy, acc, e->st);
}

// K splits of a residual-adding projection (N = hidden): with N/16 tiles
// alone too few workgroups cover the GPU, so the K range is split and the
// partial sums are added by the next RMSNorm (ec_glue_add_rmsnorm_quant).
// Measured on MI355X for N = 2560, M = 8: K 4096 5.75 -> 4.92 us (3 splits),
// K 9216 8.43 -> 6.99 us (3 splits); more splits shorten the matvec further
// but each partial adds a 10 KB row read to every RMSNorm block, and the
// decode step was fastest at 3 and 3 (EC_RESID_SPLIT="a,b" overrides the
// splits for K < 8192 and K >= 8192).
constexpr uint32_t kMaxResidSplit = 8;
uint32_t resid_split(uint32_t N, uint32_t K, int fmt = EC_Q8_0) {
    if (fmt != EC_Q8_0) return 1;
    static const std::pair<uint32_t, uint32_t> sp = [] {
        uint32_t a = 3, b = 3;
        if (const char* v = getenv("EC_RESID_SPLIT")) sscanf(v, "%u,%u", &a, &b);
        return std::make_pair(std::clamp(a, 1u, kMaxResidSplit), std::clamp(b, 1u, kMaxResidSplit));
    }();
    const uint32_t tiles = (N + 15) / 16, nG = (K + 127) / 128;
    if (tiles >= 256) return 1;
    return std::min(nG >= 64 ? sp.second : sp.first, nG);
}

// K splits of the input projection of a delta-net block and of gate/up
// (their consumers, the fused delta step and SwiGLU, add the partial sums).
// Decode step on MI355X (4B-class, batch 8, ~12k matvec waves per launch),
// one activation piece: best at 2 and 3; two pieces (two tiles per matvec
// wave): 1 and 4 (EC_IN_SPLIT / EC_GU_SPLIT override both).
uint32_t env_split(const char* name, uint32_t dflt) {
    const char* v = getenv(name);
    return std::clamp(v ? (uint32_t)atoi(v) : dflt, 1u, kMaxResidSplit);
}
// two pieces, batch 8: 1 / 2 / 3 splits 4497 / 4482 / 4476 tok/s
uint32_t in_split(uint32_t pieces) {
    static const uint32_t v[2] = {env_split("EC_IN_SPLIT", 2), env_split("EC_IN_SPLIT", 1)};
    return v[pieces == 2];
}
// gate/up (18432 x 2560), partials added by SwiGLU.  Decode batch 8 on MI355X
// with the other splits at their defaults, one piece: 2 / 3 / 4 / 5 / 6 splits
// 4632 / 4645 / 4604 / 4612 / 4553 tok/s; two pieces: 2 / 3 / 4 splits
// 4458 / 4482 / 4491 (4519 with the input projection unsplit).
uint32_t gu_split(uint32_t pieces) {
    static const uint32_t v[2] = {env_split("EC_GU_SPLIT", 3), env_split("EC_GU_SPLIT", 4)};
    return v[pieces == 2];
}
// attention input projection (q|k|v, 6144 x 2560), partials added by the rope
// kernel.  Decode batch 8 on MI355X: 1 / 2 / 3 / 4 / 5 / 6 / 8 splits
// 4623 / 4620 / 4631 / 4633 / 4633 / 4628 / 4625 tok/s.
uint32_t attn_split() {
    static const uint32_t v = env_split("EC_ATTN_SPLIT", 4);
    return v;
}

// A split count clamped to the matrix's 128-element K chunks (Q4_K: no split).
uint32_t split_count(const Mat& m, uint32_t ns) { return m.fmt == EC_Q8_0 ? std::min(ns, (m.K + 127) / 128) : 1u; }

// A split-K projection into y ([ns][B][N]); ns from split_count.  Q4_K: one
// whole-K launch into y.
int mv_split(ec_engine* e, const Mat& m, const void* act, float* y, uint32_t ns) {
    if (e->mv_bytes)  // the output counted once (the extra partial sums are not algorithmic bytes)
        e->mv_bytes->push_back((double)gguf_bytes(m, m.N) + act_alg_bytes(e, m) + (double)e->B * m.N * 4);
    if (m.fmt != EC_Q8_0) return ec_matvec_pieces(m.fmt, e->P, m.tiled, act, y, e->B, m.N, m.K, m.N, 0, e->st);
    return ec_matvec_split_pieces(EC_Q8_0, e->P, m.tiled, act, y, e->B, m.N, m.K, ns, e->st);
}

// Residual projection: ns = resid_split(m) partial sums into e->parts.
int mv_resid(ec_engine* e, const Mat& m, const void* act, uint32_t ns) { return mv_split(e, m, act, e->parts, ns); }

// Slices of the decode step's greedy pick: a row per 1024-thread workgroup
// reads ~600 KB of logits through one CU at 151936 entries; 16 slices spread
// it over 16x the CUs, merged by a second small launch.  0 = one launch (short
// vocabularies); EC_ARGMAX_SLICES overrides (0 .. 64), for comparison.
constexpr uint32_t kArgmaxSlicesMax = 64;
uint32_t argmax_slices(uint32_t vocab) {
    static const int env = [] {
        const char* v = getenv("EC_ARGMAX_SLICES");
        return v ? atoi(v) : -1;
    }();
    if (env >= 0) return std::min((uint32_t)env, kArgmaxSlicesMax);
    return vocab >= 32768 ? 16u : 0u;
}

// One launch of the decode step; with a trace callback installed, the stream
// is drained and the callback called before and after it.
template <class F>
int launch(ec_engine* e, int op, int layer, int nparts, int x_in, int x_out, F&& f) {
    if (!e->trace_cb) return f();
    ec_trace_event ev{op, layer, 0, nparts, x_in, x_out};
    EC_HIP(hipStreamSynchronize(e->st));
    e->trace_cb(e->trace_user, &ev);
    const int rc = f();
    if (rc) return rc;
    EC_HIP(hipStreamSynchronize(e->st));
    ev.phase = 1;
    e->trace_cb(e->trace_user, &ev);
    return EC_OK;
}

// The decode step (stream-ordered; captured once into a graph).  Q8_0
// matrices read the Q8_0 activations the fused glue kernels write; a Q4_K
// matrix reads a Q4_K-grouped activation quantized from the fp32 output of its
// producer (RMSNorm rows, the delta step's fp32 output, attention's output,
// SwiGLU rows), one extra launch per such input.
int record_step(ec_engine* e) {
    const ec_engine_cfg& c = e->c;
    const uint32_t B = e->B, H = e->H, F = e->F;
    hipStream_t st = e->st;
    // glue launches are left out when only the matvecs are recorded
#define EC_GLUE(op, layer, nparts, xin, xout, call)                                        \
    do {                                                                                  \
        if (!e->mv_only) EC_TRY(launch(e, op, layer, (int)(nparts), xin, xout, [&] { return (call); })); \
    } while (0)
#define EC_MV(op, layer, nparts, actb, call) EC_TRY(launch(e, op, layer, (int)(nparts), actb, -1, [&] { return (call); }))
    // xc: the current residual; ns > 0: e->parts holds ns partial sums still
    // to be added to it (by the next norm, which then moves xc to the other buffer)
    float* xc = e->x;
    uint32_t ns = 0;
    auto xid = [&](const float* p) { return p == e->x ? EC_B_X : EC_B_X2; };
    auto q4 = [](const Mat& m) { return m.fmt == EC_Q4_K; };
    // RMSNorm of the residual (adding pending partial sums first) into act_h;
    // with a Q4_K consumer also the fp32 rows and their Q4_K activation
    auto norm = [&](const float* w, int layer, bool need4) -> int {
        if (ns == 0) {
            EC_GLUE(EC_OP_NORM, layer, 0, xid(xc), xid(xc),
                    ec_glue_rmsnorm_quant_pieces(xc, w, e->act_h, B, H, e->P, st));
        } else {
            float* xn = xc == e->x ? e->x2 : e->x;
            EC_GLUE(EC_OP_NORM, layer, ns, xid(xc), xid(xn),
                    ec_glue_add_rmsnorm_quant_pieces(xc, e->parts, ns, xn, w, e->act_h, B, H, e->P, st));
            xc = xn;
            ns = 0;
        }
        if (need4) {
            EC_GLUE(EC_OP_NORM_ROWS, layer, 0, xid(xc), EC_B_HN, ec_glue_rmsnorm_rows(xc, w, e->hn, B, H, st));
            EC_GLUE(EC_OP_QUANT_ACT, layer, 0, EC_B_HN, EC_B_ACT4_H,
                    ec_quantize_act_pieces(EC_Q4_K, e->hn, e->act4_h, B, H, e->P, st));
        }
        return EC_OK;
    };
    auto ain = [&](const Mat& m, void* a8, void* a4) { return q4(m) ? a4 : a8; };
    auto aid = [&](const Mat& m, int b8, int b4) { return q4(m) ? b4 : b8; };
    EC_GLUE(EC_OP_EMBED, -1, 0, -1, EC_B_X, ec_glue_embed_fmt(e->embed_fmt, e->embed, e->tok, e->x, B, H, c.vocab, st));
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        Layer& y = e->L[l];
        const int li = (int)l;
        EC_TRY(norm(y.attn_norm, li, q4(y.w_in)));
        if (!y.attn) {
            const uint32_t Nin = e->nin_delta;
            const uint32_t nsi = split_count(y.w_in, in_split(e->P));
            EC_MV(EC_OP_MV_IN, li, nsi, aid(y.w_in, EC_B_ACT_H, EC_B_ACT4_H),
                  mv_split(e, y.w_in, ain(y.w_in, e->act_h, e->act4_h), e->proj, nsi));
            // conv + gates + delta rule + gated norm + quantize in one launch
            // (fp32 output instead when the output projection is Q4_K)
            const bool o4 = q4(y.w_out);
            EC_GLUE(EC_OP_DELTA_STEP, li, nsi, -1, o4 ? EC_B_CORE : EC_B_ACT_V,
                    ec_delta_step_out_pieces(e->proj, nsi, Nin, y.conv_state, y.conv_w, y.a_log, y.dt_bias,
                                             y.ssm_norm, y.ssm_state, o4 ? nullptr : e->act_v,
                                             o4 ? e->core_f : nullptr, e->pos, B, e->n_k, e->n_v, c.conv_kernel, e->P,
                                             st));
            if (o4)
                EC_GLUE(EC_OP_QUANT_ACT, li, 0, EC_B_CORE, EC_B_ACT4_V,
                        ec_quantize_act_pieces(EC_Q4_K, e->core_f, e->act4_v, B, e->value_dim, e->P, st));
            ns = resid_split(y.w_out.N, y.w_out.K, y.w_out.fmt);
            EC_MV(EC_OP_MV_OUT, li, ns, aid(y.w_out, EC_B_ACT_V, EC_B_ACT4_V),
                  mv_resid(e, y.w_out, ain(y.w_out, e->act_v, e->act4_v), ns));
        } else {
            const uint32_t Nin = e->nin_attn;
            const uint32_t nsa = split_count(y.w_in, attn_split());
            EC_MV(EC_OP_MV_IN, li, nsa, aid(y.w_in, EC_B_ACT_H, EC_B_ACT4_H),
                  mv_split(e, y.w_in, ain(y.w_in, e->act_h, e->act4_h), e->proj, nsa));
            const bool o4 = q4(y.w_out);
            if (e->packed_attn) {
                // rope + KV append write q as int8 pieces; attention writes the
                // Q8_0 activation of its output for the output projection
                EC_GLUE(EC_OP_ROPE_APPEND, li, nsa, -1, -1,
                        ec_glue_qk_rope_append_split(e->proj, nsa, Nin, y.q_norm, y.k_norm, y.use_qn, y.use_kn,
                                                     e->inv_freq, e->pos, nullptr, e->q_packed, e->q_scales, y.keys,
                                                     y.vals, y.ks, y.vs, e->ctx, B, e->seq_stride, c.max_ctx,
                                                     c.n_heads, c.n_kv, c.head_dim, st));
                EC_GLUE(EC_OP_ATTN, li, 0, -1, o4 ? -1 : EC_B_ACT_Q,
                        ec_attn_decode_packed_pieces(e->q_packed, e->q_scales, y.keys, y.vals, y.ks, y.vs,
                                                     e->attn_out, o4 ? nullptr : e->act_q, e->ctx, B, e->seq_stride,
                                                     c.n_heads, c.n_kv, c.max_ctx, e->P, e->attn_ws, st));
            } else {
                EC_GLUE(EC_OP_ROPE_APPEND, li, nsa, -1, -1,
                        ec_glue_qk_rope_append_split(e->proj, nsa, Nin, y.q_norm, y.k_norm, y.use_qn, y.use_kn,
                                                     e->inv_freq, e->pos, e->qbuf, nullptr, nullptr, y.keys, y.vals,
                                                     y.ks, y.vs, e->ctx, B, e->seq_stride, c.max_ctx, c.n_heads,
                                                     c.n_kv, c.head_dim, st));
                EC_GLUE(EC_OP_ATTN, li, 0, -1, -1,
                        ec_attn_decode(e->qbuf, y.keys, y.vals, y.ks, y.vs, e->attn_out, e->ctx, B, e->seq_stride,
                                       c.n_heads, c.n_kv, c.head_dim, c.max_ctx, e->attn_ws, st));
                if (!o4)
                    EC_GLUE(EC_OP_QUANT_ACT, li, 0, EC_B_ATTN_OUT, EC_B_ACT_Q,
                            ec_quantize_act_pieces(EC_Q8_0, e->attn_out, e->act_q, B, e->q_dim, e->P, st));
            }
            if (o4)
                EC_GLUE(EC_OP_QUANT_ACT, li, 0, EC_B_ATTN_OUT, EC_B_ACT4_Q,
                        ec_quantize_act_pieces(EC_Q4_K, e->attn_out, e->act4_q, B, e->q_dim, e->P, st));
            ns = resid_split(y.w_out.N, y.w_out.K, y.w_out.fmt);
            EC_MV(EC_OP_MV_OUT, li, ns, aid(y.w_out, EC_B_ACT_Q, EC_B_ACT4_Q),
                  mv_resid(e, y.w_out, ain(y.w_out, e->act_q, e->act4_q), ns));
        }
        EC_TRY(norm(y.ffn_norm, li, q4(y.w_gu)));
        const bool d4 = q4(y.w_down);
        // a Q4_K down projection reads SwiGLU rows, which take one gate/up part
        const uint32_t nsg = d4 ? 1u : split_count(y.w_gu, gu_split(e->P));
        EC_MV(EC_OP_MV_GU, li, nsg, aid(y.w_gu, EC_B_ACT_H, EC_B_ACT4_H),
              mv_split(e, y.w_gu, ain(y.w_gu, e->act_h, e->act4_h), e->gu, nsg));
        if (d4) {
            EC_GLUE(EC_OP_SWIGLU, li, nsg, -1, EC_B_FF, ec_glue_swiglu_rows(e->gu, e->ff, B, F, st));
            EC_GLUE(EC_OP_QUANT_ACT, li, 0, EC_B_FF, EC_B_ACT4_F,
                    ec_quantize_act_pieces(EC_Q4_K, e->ff, e->act4_f, B, F, e->P, st));
        } else {
            EC_GLUE(EC_OP_SWIGLU, li, nsg, -1, EC_B_ACT_F,
                    ec_glue_swiglu_quant_split_pieces(e->gu, nsg, e->act_f, B, F, e->P, st));
        }
        ns = resid_split(y.w_down.N, y.w_down.K, y.w_down.fmt);
        EC_MV(EC_OP_MV_DOWN, li, ns, aid(y.w_down, EC_B_ACT_F, EC_B_ACT4_F),
              mv_resid(e, y.w_down, ain(y.w_down, e->act_f, e->act4_f), ns));
    }
    EC_TRY(norm(e->final_norm, -1, q4(e->lm_head)));
    EC_MV(EC_OP_LM_HEAD, -1, 0, aid(e->lm_head, EC_B_ACT_H, EC_B_ACT4_H),
          mv(e, e->lm_head, ain(e->lm_head, e->act_h, e->act4_h), e->logits, c.vocab, 0));
    const uint32_t nsl = argmax_slices(c.vocab);
    EC_GLUE(EC_OP_ARGMAX, -1, 0, -1, -1,
            nsl ? ec_glue_argmax_advance_sliced(e->logits, c.vocab, e->gen, e->tok, e->pos, B, c.max_ctx, nsl,
                                                e->am_ws, st)
                : ec_glue_argmax_advance_bounded(e->logits, c.vocab, e->gen, e->tok, e->pos, B, c.max_ctx, st));
    return EC_OK;
#undef EC_GLUE
#undef EC_MV
}

int destroy_graph(ec_engine* e) {
    if (e->exec) (void)hipGraphExecDestroy(e->exec);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    e->exec = nullptr;
    e->graph = nullptr;
    return EC_OK;
}

}  // namespace

extern "C" int ec_engine_create(const ec_engine_cfg* cfg, ec_engine** out) {
    if (!cfg || !out) return ec_set_error(EC_ERR_ARG, "ec_engine_create: null argument");
    const ec_engine_cfg& c = *cfg;
    // ssm_heads == 0: no delta-net blocks (every block attention, attn_interval 1)
    const bool delta_ok = c.ssm_heads == 0 ? (c.ssm_inner == 0 && c.attn_interval == 1)
                                           : (c.ssm_inner == c.ssm_heads * 128 && c.ssm_inner % 256 == 0 &&
                                              c.conv_kernel != 0 && c.attn_interval != 0);
    if (c.hidden % 128 || c.ffn % 128 || c.head_dim != 256 || c.n_kv == 0 || c.n_heads % c.n_kv || !delta_ok ||
        c.max_batch == 0 || c.max_batch > 16 || c.max_ctx == 0 || c.vocab == 0)
        return ec_set_error(EC_ERR_ARG,
                            "ec_engine_create: need hidden, ffn % 128 == 0, head_dim 256, ssm_inner = 128*ssm_heads "
                            "(or both 0 with attn_interval 1), 1 <= max_batch <= 16");
    ec_engine* e = new ec_engine();
    e->c = c;
    e->B = c.max_batch;
    e->H = c.hidden;
    e->F = c.ffn;
    e->q_dim = c.n_heads * c.head_dim;
    e->kv_dim = c.n_kv * c.head_dim;
    e->value_dim = c.ssm_inner;
    e->key_dim = c.ssm_inner / 2;  // qwen_linear.zig:117-119
    e->n_v = c.ssm_heads;
    e->n_k = e->key_dim / 128;
    e->conv_dim = 2 * e->key_dim + e->value_dim;
    e->nin_delta = e->conv_dim + e->value_dim + 2 * e->n_v;
    e->nin_attn = e->q_dim + 2 * e->kv_dim;
    e->nin_max = std::max(e->nin_delta, e->nin_attn);
    // A whole multiple of 64 positions per sequence puts every sequence's row p
    // at the same offset modulo a large power of two; four spare positions
    // break that (batch 8, 4096 positions, 128-position attention chunks:
    // 19.7 -> 17.8 us per launch on MI355X; 8192: 20.7 -> 17.8).
    e->ctx_stride = c.max_ctx % 64 == 0 ? c.max_ctx + 4 : c.max_ctx;
    e->seq_stride = (uint64_t)e->ctx_stride * e->kv_dim;
    int rc = EC_OK;
    auto fail = [&](int r) {
        ec_engine_destroy(e);
        return r;
    };
    if (hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking) != hipSuccess)
        return fail(ec_set_error(EC_ERR_HIP, "ec_engine_create: stream"));
    const uint32_t B = e->B, H = e->H;
    e->L.resize(c.n_layers);
    size_t wb = 0;
    for (uint32_t l = 0; l < c.n_layers && rc == EC_OK; ++l) {
        Layer& y = e->L[l];
        y.attn = is_attn(c, l);
        const uint32_t Nin = y.attn ? e->nin_attn : e->nin_delta;
        const uint32_t Kout = y.attn ? e->q_dim : e->value_dim;
        if ((rc = alloc_mat(e, y.w_in, Nin, H)) || (rc = alloc_mat(e, y.w_out, H, Kout)) ||
            (rc = alloc_mat(e, y.w_gu, 2 * e->F, H)) || (rc = alloc_mat(e, y.w_down, H, e->F)) ||
            (rc = dalloc(e, &y.attn_norm, H)) || (rc = dalloc(e, &y.ffn_norm, H)))
            break;
        wb += 2 * H * 4;
        if (!y.attn) {
            if ((rc = dalloc(e, &y.conv_w, (size_t)c.conv_kernel * e->conv_dim)) ||
                (rc = dalloc(e, &y.a_log, e->n_v)) || (rc = dalloc(e, &y.dt_bias, e->n_v)) ||
                (rc = dalloc(e, &y.ssm_norm, 128)) ||
                (rc = dalloc(e, &y.conv_state, (size_t)B * c.conv_kernel * e->conv_dim)) ||
                (rc = dalloc(e, &y.ssm_state, (size_t)B * e->n_v * 128 * 128)))
                break;
            wb += ((size_t)c.conv_kernel * e->conv_dim + 2 * e->n_v + 128) * 4;
        } else {
            if ((rc = dalloc(e, &y.q_norm, c.head_dim)) || (rc = dalloc(e, &y.k_norm, c.head_dim)) ||
                (rc = dalloc(e, &y.keys, (size_t)B * e->seq_stride)) ||
                (rc = dalloc(e, &y.vals, (size_t)B * e->seq_stride)) ||
                (rc = dalloc(e, &y.ks, (size_t)B * e->ctx_stride * c.n_kv)) ||
                (rc = dalloc(e, &y.vs, (size_t)B * e->ctx_stride * c.n_kv)))
                break;
            wb += 2 * c.head_dim * 4;
        }
    }
    if (rc) return fail(rc);
    wb += H * 4;
    e->weight_bytes = wb;  // vectors; the matrices are counted by ec_engine_weight_bytes
    if ((rc = dalloc(e, &e->embed, embed_bytes(e))) || (rc = dalloc(e, &e->final_norm, H)) ||
        (rc = alloc_mat(e, e->lm_head, c.vocab, H)) || (rc = dalloc(e, &e->x, (size_t)B * H)) ||
        (rc = dalloc(e, &e->x2, (size_t)B * H)) || (rc = dalloc(e, &e->parts, (size_t)kMaxResidSplit * B * H)) ||
        (rc = dalloc(e, &e->proj, (size_t)kMaxResidSplit * B * e->nin_max)) ||
        (rc = dalloc(e, &e->gu, (size_t)kMaxResidSplit * B * 2 * e->F)) ||
        (rc = dalloc(e, &e->core, (size_t)B * e->value_dim)) || (rc = dalloc(e, &e->q, (size_t)B * e->key_dim)) ||
        (rc = dalloc(e, &e->k, (size_t)B * e->key_dim)) || (rc = dalloc(e, &e->v, (size_t)B * e->value_dim)) ||
        (rc = dalloc(e, &e->dec, (size_t)B * e->n_v)) || (rc = dalloc(e, &e->beta, (size_t)B * e->n_v)) ||
        (rc = dalloc(e, &e->qbuf, (size_t)B * e->q_dim)) || (rc = dalloc(e, &e->attn_out, (size_t)B * e->q_dim)) ||
        (rc = dalloc(e, &e->logits, (size_t)B * c.vocab)) || (rc = dalloc(e, &e->inv_freq, c.head_dim / 2)) ||
        (rc = dalloc(e, &e->am_ws, ec_glue_argmax_ws_bytes(B, kArgmaxSlicesMax))) ||
        (rc = dalloc(e, &e->act_h, ec_act_bytes_pieces(EC_Q8_0, B, H, 2))) ||
        (rc = dalloc(e, &e->act_v, ec_act_bytes_pieces(EC_Q8_0, B, e->value_dim, 2))) ||
        (rc = dalloc(e, &e->act_f, ec_act_bytes_pieces(EC_Q8_0, B, e->F, 2))) ||
        (rc = dalloc(e, &e->act_q, ec_act_bytes_pieces(EC_Q8_0, B, e->q_dim, 2))) ||
        (rc = dalloc(e, &e->attn_ws, ec_attn_ws_bytes(B, c.n_heads, c.head_dim, c.max_ctx))) ||
        (rc = dalloc(e, &e->tok, B)) || (rc = dalloc(e, &e->pos, B)) || (rc = dalloc(e, &e->gen, B)) ||
        (rc = dalloc(e, &e->ctx, B)))
        return fail(rc);
    const uint32_t G = c.n_heads / c.n_kv;
    e->packed_attn = c.head_dim == 256 && (G == 1 || G == 2 || G == 4);
    if (e->packed_attn && ((rc = dalloc(e, &e->q_packed, ec_attn_qa_bytes(B, c.n_heads))) ||
                           (rc = dalloc(e, &e->q_scales, (size_t)B * c.n_heads * 3))))
        return fail(rc);
    if (hipHostMalloc((void**)&e->h_io, (size_t)ec_engine::kIoSlots * 32 * sizeof(int32_t)) != hipSuccess)
        return fail(ec_set_error(EC_ERR_HIP, "ec_engine_create: pinned buffer"));
    for (hipEvent_t& ev : e->io_ev)
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
            return fail(ec_set_error(EC_ERR_HIP, "ec_engine_create: event"));
    // RoPE inverse frequencies, 1/pow(base, i/head_dim) in fp32 (engine.zig:476)
    std::vector<float> inv(c.head_dim / 2);
    for (uint32_t i = 0; i < c.head_dim; i += 2)
        inv[i / 2] = 1.0f / powf(c.rope_base, (float)i / (float)c.head_dim);
    if ((rc = upload_vec(e, e->inv_freq, inv))) return fail(rc);
    std::vector<int32_t> neg(B, -1);
    if ((rc = h2d(e, e->pos, neg.data(), B * 4))) return fail(rc);
    *out = e;
    return EC_OK;
}

extern "C" int ec_engine_get_config(const ec_engine* e, ec_engine_cfg* out) {
    if (!e || !out) return ec_set_error(EC_ERR_ARG, "ec_engine_get_config: null argument");
    *out = e->c;
    return EC_OK;
}

namespace {

// The matrix a (layer, tensor) names, or nullptr.
Mat* find_mat(ec_engine* e, int layer, int tensor) {
    if (tensor == EC_T_LM_HEAD) return &e->lm_head;
    if (layer < 0 || layer >= (int)e->c.n_layers) return nullptr;
    Layer& y = e->L[layer];
    switch (tensor) {
        case EC_T_W_IN: return &y.w_in;
        case EC_T_W_OUT: return &y.w_out;
        case EC_T_W_GATE:
        case EC_T_W_UP: return &y.w_gu;
        case EC_T_W_DOWN: return &y.w_down;
        default: return nullptr;
    }
}

// Buffers of Q4_K inputs, allocated with the first Q4_K matrix.
int alloc_q4(ec_engine* e) {
    if (e->q4) return EC_OK;
    const uint32_t B = e->B;
    EC_TRY(dalloc(e, &e->hn, (size_t)B * e->H));
    EC_TRY(dalloc(e, &e->core_f, (size_t)B * std::max(e->value_dim, 1u)));
    EC_TRY(dalloc(e, &e->ff, (size_t)B * e->F));
    EC_TRY(dalloc(e, &e->act4_h, ec_act_bytes_pieces(EC_Q4_K, B, e->H, 2)));
    EC_TRY(dalloc(e, &e->act4_v, e->value_dim % 256 ? 16 : ec_act_bytes_pieces(EC_Q4_K, B, e->value_dim, 2)));
    EC_TRY(dalloc(e, &e->act4_q, ec_act_bytes_pieces(EC_Q4_K, B, e->q_dim, 2)));
    EC_TRY(dalloc(e, &e->act4_f, e->F % 256 ? 16 : ec_act_bytes_pieces(EC_Q4_K, B, e->F, 2)));
    e->q4 = true;
    return EC_OK;
}

// Free one allocation the engine owns (and forget it).
void dfree(ec_engine* e, void* p) {
    auto it = std::find(e->allocs.begin(), e->allocs.end(), p);
    if (it != e->allocs.end()) e->allocs.erase(it);
    (void)hipFree(p);
}

}  // namespace

extern "C" int ec_engine_set_format(ec_engine* e, int layer, int tensor, int fmt) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_set_format: null engine");
    EC_HIP(hipStreamSynchronize(e->st));
    if (tensor == EC_T_EMBED) {
        if (fmt != EC_Q8_0 && fmt != EC_F16 && fmt != EC_F32)
            return ec_set_error(EC_ERR_UNSUPPORTED, "ec_engine_set_format: embedding is Q8_0, F16 or F32");
        if (fmt == e->embed_fmt) return EC_OK;
        dfree(e, e->embed);
        e->embed = nullptr;
        e->embed_fmt = fmt;
        destroy_graph(e);
        return dalloc(e, &e->embed, embed_bytes(e));
    }
    Mat* m = find_mat(e, layer, tensor);
    if (!m) return ec_set_error(EC_ERR_ARG, "ec_engine_set_format: not a matrix tensor");
    if (fmt != EC_Q8_0 && fmt != EC_Q4_K)
        return ec_set_error(EC_ERR_UNSUPPORTED, "ec_engine_set_format: matrices are Q8_0 or Q4_K");
    if (fmt == EC_Q4_K && m->K % 256)
        return ec_set_error(EC_ERR_ARG, "ec_engine_set_format: Q4_K needs K % 256 == 0");
    if (fmt == m->fmt) return EC_OK;
    if (fmt == EC_Q4_K) EC_TRY(alloc_q4(e));
    dfree(e, m->tiled);
    m->tiled = nullptr;
    m->fmt = fmt;
    destroy_graph(e);
    return dalloc(e, &m->tiled, ec_tiled_bytes(fmt, m->N, m->K));
}

extern "C" int ec_engine_set_act_pieces(ec_engine* e, uint32_t pieces) {
    if (!e || (pieces != 1 && pieces != 2)) return ec_set_error(EC_ERR_ARG, "ec_engine_set_act_pieces: 1 or 2 pieces");
    if (pieces == e->P) return EC_OK;
    EC_HIP(hipStreamSynchronize(e->st));
    e->P = pieces;
    return destroy_graph(e);
}

extern "C" int ec_engine_get_act_pieces(const ec_engine* e) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_get_act_pieces: null engine");
    return (int)e->P;
}

extern "C" int ec_engine_get_format(const ec_engine* e, int layer, int tensor) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_get_format: null engine");
    if (tensor == EC_T_EMBED) return e->embed_fmt;
    const Mat* m = find_mat(const_cast<ec_engine*>(e), layer, tensor);
    if (!m) return ec_set_error(EC_ERR_ARG, "ec_engine_get_format: not a matrix tensor");
    return m->fmt;
}

extern "C" void ec_engine_destroy(ec_engine* e) {
    if (!e) return;
    if (e->st) (void)hipStreamSynchronize(e->st);
    for (uint32_t i = 1; i < ec_engine::kPrefillLanes; ++i)
        if (e->pf[i].st) {
            (void)hipStreamSynchronize(e->pf[i].st);
            (void)hipStreamDestroy(e->pf[i].st);
        }
    destroy_graph(e);
    for (void* p : e->allocs) (void)hipFree(p);
    if (e->h_io) (void)hipHostFree(e->h_io);
    for (hipEvent_t ev : e->io_ev)
        if (ev) (void)hipEventDestroy(ev);
    if (e->st) (void)hipStreamDestroy(e->st);
    delete e;
}

extern "C" int ec_engine_set_tensor(ec_engine* e, int layer, int tensor, const void* host, size_t bytes) {
    if (!e || !host) return ec_set_error(EC_ERR_ARG, "ec_engine_set_tensor: null argument");
    const ec_engine_cfg& c = e->c;
    auto need = [&](size_t n) -> int {
        if (bytes != n) {
            char buf[160];
            snprintf(buf, sizeof buf, "ec_engine_set_tensor(%d, %d): %zu bytes given, %zu expected", layer, tensor,
                     bytes, n);
            return ec_set_error(EC_ERR_ARG, buf);
        }
        return EC_OK;
    };
    auto vec = [&](float* dst, size_t n) -> int {
        EC_TRY(need(n * 4));
        return h2d(e, dst, host, bytes);
    };
    if (tensor == EC_T_EMBED) {
        EC_TRY(need(embed_bytes(e)));
        return h2d(e, e->embed, host, bytes);
    }
    if (tensor == EC_T_FINAL_NORM) return vec(e->final_norm, e->H);
    if (tensor == EC_T_LM_HEAD) {
        EC_TRY(need(gguf_bytes(e->lm_head, c.vocab)));
        return upload_rows(e, e->lm_head, 0, host, c.vocab);
    }
    if (layer < 0 || (uint32_t)layer >= c.n_layers) return ec_set_error(EC_ERR_ARG, "ec_engine_set_tensor: layer");
    Layer& y = e->L[layer];
    destroy_graph(e);  // weights are captured by address only, but keep the rule simple
    switch (tensor) {
        case EC_T_ATTN_NORM: return vec(y.attn_norm, e->H);
        case EC_T_FFN_NORM: return vec(y.ffn_norm, e->H);
        case EC_T_W_IN: EC_TRY(need(gguf_bytes(y.w_in, y.w_in.N))); return upload_rows(e, y.w_in, 0, host, y.w_in.N);
        case EC_T_W_OUT: EC_TRY(need(gguf_bytes(y.w_out, e->H))); return upload_rows(e, y.w_out, 0, host, e->H);
        case EC_T_W_GATE: EC_TRY(need(gguf_bytes(y.w_gu, e->F))); return upload_rows(e, y.w_gu, 0, host, e->F);
        case EC_T_W_UP: EC_TRY(need(gguf_bytes(y.w_gu, e->F))); return upload_rows(e, y.w_gu, e->F, host, e->F);
        case EC_T_W_DOWN: EC_TRY(need(gguf_bytes(y.w_down, e->H))); return upload_rows(e, y.w_down, 0, host, e->H);
        default: break;
    }
    if (!y.attn) {
        switch (tensor) {
            case EC_T_CONV_W: return vec(y.conv_w, (size_t)c.conv_kernel * e->conv_dim);
            case EC_T_A_LOG: return vec(y.a_log, e->n_v);
            case EC_T_DT_BIAS: return vec(y.dt_bias, e->n_v);
            case EC_T_SSM_NORM: return vec(y.ssm_norm, 128);
            default: break;
        }
    } else if (tensor == EC_T_Q_NORM || tensor == EC_T_K_NORM) {
        EC_TRY(need((size_t)c.head_dim * 4));
        const float* f = (const float*)host;
        int nz = 0;
        for (uint32_t i = 0; i < c.head_dim; ++i) nz |= f[i] != 0.0f;
        (tensor == EC_T_Q_NORM ? y.use_qn : y.use_kn) = nz;
        return vec(tensor == EC_T_Q_NORM ? y.q_norm : y.k_norm, c.head_dim);
    }
    return ec_set_error(EC_ERR_ARG, "ec_engine_set_tensor: tensor id not valid for this layer");
}

namespace {
int download_rows(ec_engine* e, const Mat& m, uint32_t row0, void* host, uint32_t N) {
    void* tmp = nullptr;
    EC_HIP(hipMalloc(&tmp, gguf_bytes(m, N)));
    const uint8_t* src = (const uint8_t*)m.tiled + ec_tiled_bytes(m.fmt, row0, m.K);
    int rc = ec_unpack_tiled(m.fmt, src, tmp, N, m.K, e->st);
    if (!rc && hipMemcpyAsync(host, tmp, gguf_bytes(m, N), hipMemcpyDeviceToHost, e->st) != hipSuccess)
        rc = ec_set_error(EC_ERR_HIP, "download_rows: copy");
    (void)hipStreamSynchronize(e->st);
    (void)hipFree(tmp);
    return rc;
}
}  // namespace

extern "C" int ec_engine_get_tensor(ec_engine* e, int layer, int tensor, void* host, size_t bytes) {
    if (!e || !host) return ec_set_error(EC_ERR_ARG, "ec_engine_get_tensor: null argument");
    const ec_engine_cfg& c = e->c;
    auto need = [&](size_t n) -> int {
        return bytes == n ? EC_OK : ec_set_error(EC_ERR_ARG, "ec_engine_get_tensor: wrong byte count");
    };
    auto vec = [&](const float* src, size_t n) -> int {
        EC_TRY(need(n * 4));
        return d2h(e, host, src, bytes);
    };
    if (tensor == EC_T_EMBED) {
        EC_TRY(need(embed_bytes(e)));
        return d2h(e, host, e->embed, bytes);
    }
    if (tensor == EC_T_FINAL_NORM) return vec(e->final_norm, e->H);
    if (tensor == EC_T_LM_HEAD) {
        EC_TRY(need(gguf_bytes(e->lm_head, c.vocab)));
        return download_rows(e, e->lm_head, 0, host, c.vocab);
    }
    if (layer < 0 || (uint32_t)layer >= c.n_layers) return ec_set_error(EC_ERR_ARG, "ec_engine_get_tensor: layer");
    const Layer& y = e->L[layer];
    switch (tensor) {
        case EC_T_ATTN_NORM: return vec(y.attn_norm, e->H);
        case EC_T_FFN_NORM: return vec(y.ffn_norm, e->H);
        case EC_T_W_IN: EC_TRY(need(gguf_bytes(y.w_in, y.w_in.N))); return download_rows(e, y.w_in, 0, host, y.w_in.N);
        case EC_T_W_OUT: EC_TRY(need(gguf_bytes(y.w_out, e->H))); return download_rows(e, y.w_out, 0, host, e->H);
        case EC_T_W_GATE: EC_TRY(need(gguf_bytes(y.w_gu, e->F))); return download_rows(e, y.w_gu, 0, host, e->F);
        case EC_T_W_UP: EC_TRY(need(gguf_bytes(y.w_gu, e->F))); return download_rows(e, y.w_gu, e->F, host, e->F);
        case EC_T_W_DOWN: EC_TRY(need(gguf_bytes(y.w_down, e->H))); return download_rows(e, y.w_down, 0, host, e->H);
        default: break;
    }
    if (!y.attn) {
        switch (tensor) {
            case EC_T_CONV_W: return vec(y.conv_w, (size_t)c.conv_kernel * e->conv_dim);
            case EC_T_A_LOG: return vec(y.a_log, e->n_v);
            case EC_T_DT_BIAS: return vec(y.dt_bias, e->n_v);
            case EC_T_SSM_NORM: return vec(y.ssm_norm, 128);
            default: break;
        }
    } else if (tensor == EC_T_Q_NORM) {
        return vec(y.q_norm, c.head_dim);
    } else if (tensor == EC_T_K_NORM) {
        return vec(y.k_norm, c.head_dim);
    }
    return ec_set_error(EC_ERR_ARG, "ec_engine_get_tensor: tensor id not valid for this layer");
}

extern "C" int ec_engine_get_state(ec_engine* e, int layer, int which, uint32_t seq, void* host, size_t bytes) {
    if (!e || !host) return ec_set_error(EC_ERR_ARG, "ec_engine_get_state: null argument");
    const ec_engine_cfg& c = e->c;
    if (layer < 0 || (uint32_t)layer >= c.n_layers || seq >= e->B)
        return ec_set_error(EC_ERR_ARG, "ec_engine_get_state: layer or sequence out of range");
    const Layer& y = e->L[layer];
    const void* src = nullptr;
    size_t n = 0;
    if (!y.attn && which == EC_S_CONV) {
        n = (size_t)c.conv_kernel * e->conv_dim * 4;
        src = y.conv_state + (size_t)seq * c.conv_kernel * e->conv_dim;
    } else if (!y.attn && which == EC_S_SSM) {
        n = (size_t)e->n_v * 128 * 128 * 4;
        src = y.ssm_state + (size_t)seq * e->n_v * 128 * 128;
    } else if (y.attn && (which == EC_S_KEYS || which == EC_S_VALS)) {
        n = (size_t)c.max_ctx * e->kv_dim;  // the first max_ctx positions of the sequence's stride
        src = (which == EC_S_KEYS ? y.keys : y.vals) + (size_t)seq * e->seq_stride;
    } else if (y.attn && (which == EC_S_KSCALES || which == EC_S_VSCALES)) {
        n = (size_t)c.max_ctx * c.n_kv * 4;
        src = (which == EC_S_KSCALES ? y.ks : y.vs) + (size_t)seq * e->ctx_stride * c.n_kv;
    } else {
        return ec_set_error(EC_ERR_ARG, "ec_engine_get_state: state id not valid for this layer");
    }
    if (bytes != n) return ec_set_error(EC_ERR_ARG, "ec_engine_get_state: wrong byte count");
    return d2h(e, host, src, n);
}

extern "C" int ec_engine_init_random(ec_engine* e, uint64_t seed, float w_scale) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_init_random: null engine");
    const ec_engine_cfg& c = e->c;
    destroy_graph(e);
    if (e->embed_fmt != EC_Q8_0) return ec_set_error(EC_ERR_UNSUPPORTED, "ec_engine_init_random: Q8_0 tensors only");
    size_t tmp_bytes = gguf_bytes(EC_Q8_0, c.vocab, e->H);
    for (const Layer& y : e->L)
        tmp_bytes = std::max(tmp_bytes, std::max(gguf_bytes(EC_Q8_0, y.w_in.N, e->H), gguf_bytes(EC_Q8_0, e->F, e->H)));
    void* tmp = nullptr;
    EC_HIP(hipMalloc(&tmp, tmp_bytes));
    uint64_t stream_id = 0;
    auto next_seed = [&]() { return sm64(seed, stream_id++); };
    int rc = EC_OK;
    // embedding (GGUF rows, looked up in place) and the output head
    rc = ec_fill_random(1, e->embed, (uint64_t)c.vocab * (e->H / 32), next_seed(), w_scale, e->H, e->st);
    if (!rc) rc = random_rows(e, e->lm_head, 0, c.vocab, next_seed(), w_scale, tmp);
    if (!rc) rc = upload_vec(e, e->final_norm, gen_vec(next_seed(), e->H, 1.0, 0.1));
    for (uint32_t l = 0; l < c.n_layers && !rc; ++l) {
        Layer& y = e->L[l];
        rc = random_rows(e, y.w_in, 0, y.w_in.N, next_seed(), w_scale, tmp);
        if (!rc) rc = random_rows(e, y.w_out, 0, e->H, next_seed(), w_scale, tmp);
        if (!rc) rc = random_rows(e, y.w_gu, 0, e->F, next_seed(), w_scale, tmp);
        if (!rc) rc = random_rows(e, y.w_gu, e->F, e->F, next_seed(), w_scale, tmp);
        if (!rc) rc = random_rows(e, y.w_down, 0, e->H, next_seed(), w_scale, tmp);
        if (!rc) rc = upload_vec(e, y.attn_norm, gen_vec(next_seed(), e->H, 1.0, 0.1));
        if (!rc) rc = upload_vec(e, y.ffn_norm, gen_vec(next_seed(), e->H, 1.0, 0.1));
        if (rc) break;
        if (!y.attn) {
            rc = upload_vec(e, y.conv_w, gen_vec(next_seed(), (size_t)c.conv_kernel * e->conv_dim, 0.0, 0.5));
            std::vector<float> al(e->n_v);
            const uint64_t sa = next_seed();
            for (uint32_t h = 0; h < e->n_v; ++h) al[h] = (float)std::log(1.0 + 15.0 * u01(sm64(sa, h)));
            if (!rc) rc = upload_vec(e, y.a_log, al);
            if (!rc) rc = upload_vec(e, y.dt_bias, gen_vec(next_seed(), e->n_v, 0.0, 0.1));
            if (!rc) rc = upload_vec(e, y.ssm_norm, gen_vec(next_seed(), 128, 1.0, 0.1));
        } else {
            rc = upload_vec(e, y.q_norm, gen_vec(next_seed(), c.head_dim, 1.0, 0.1));
            if (!rc) rc = upload_vec(e, y.k_norm, gen_vec(next_seed(), c.head_dim, 1.0, 0.1));
            y.use_qn = y.use_kn = 1;
        }
        if (!rc && hipStreamSynchronize(e->st) != hipSuccess) rc = ec_set_error(EC_ERR_HIP, "init_random: sync");
    }
    (void)hipStreamSynchronize(e->st);
    (void)hipFree(tmp);
    return rc;
}

extern "C" int ec_engine_reset(ec_engine* e) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_reset: null engine");
    const ec_engine_cfg& c = e->c;
    for (Layer& y : e->L) {
        if (!y.attn) {
            EC_HIP(hipMemsetAsync(y.conv_state, 0, (size_t)e->B * c.conv_kernel * e->conv_dim * 4, e->st));
            EC_HIP(hipMemsetAsync(y.ssm_state, 0, (size_t)e->B * e->n_v * 128 * 128 * 4, e->st));
        } else {
            EC_HIP(hipMemsetAsync(y.keys, 0, (size_t)e->B * e->seq_stride, e->st));
            EC_HIP(hipMemsetAsync(y.vals, 0, (size_t)e->B * e->seq_stride, e->st));
            EC_HIP(hipMemsetAsync(y.ks, 0, (size_t)e->B * e->ctx_stride * c.n_kv * 4, e->st));
            EC_HIP(hipMemsetAsync(y.vs, 0, (size_t)e->B * e->ctx_stride * c.n_kv * 4, e->st));
        }
    }
    std::vector<int32_t> neg(e->B, -1);
    EC_HIP(hipMemcpyAsync(e->pos, neg.data(), e->B * 4, hipMemcpyHostToDevice, e->st));
    EC_HIP(hipStreamSynchronize(e->st));
    return EC_OK;
}

extern "C" int ec_engine_set_inputs(ec_engine* e, const int32_t* tok, const int32_t* pos, uint32_t n) {
    if (!e || !tok || !pos || n > e->B) return ec_set_error(EC_ERR_ARG, "ec_engine_set_inputs: bad argument");
    for (uint32_t i = 0; i < e->B; ++i) {
        const bool in = i < n;
        const int32_t t = in ? tok[i] : 0;
        if (t < 0 || (uint32_t)t >= e->c.vocab) return ec_set_error(EC_ERR_ARG, "ec_engine_set_inputs: token id");
        const int32_t p = in ? pos[i] : -1;
        if (p >= 0 && (uint32_t)p >= e->c.max_ctx) return ec_set_error(EC_ERR_ARG, "ec_engine_set_inputs: KV cache full");
    }
    const uint32_t slot = e->io_next;
    e->io_next = (slot + 1) % ec_engine::kIoSlots;
    if (e->io_pending[slot]) EC_HIP(hipEventSynchronize(e->io_ev[slot]));
    int32_t* h = e->h_io + (size_t)slot * 32;
    for (uint32_t i = 0; i < e->B; ++i) {
        h[i] = i < n ? tok[i] : 0;
        h[16 + i] = i < n ? pos[i] : -1;
    }
    EC_HIP(hipMemcpyAsync(e->tok, h, e->B * 4, hipMemcpyHostToDevice, e->st));
    EC_HIP(hipMemcpyAsync(e->pos, h + 16, e->B * 4, hipMemcpyHostToDevice, e->st));
    EC_HIP(hipEventRecord(e->io_ev[slot], e->st));
    e->io_pending[slot] = true;
    return EC_OK;
}

extern "C" int ec_engine_step(ec_engine* e, int use_graph) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_step: null engine");
    if (!use_graph) return record_step(e);
    if (!e->exec) {
        EC_HIP(hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
        int rc = record_step(e);
        hipGraph_t g = nullptr;
        hipError_t ce = hipStreamEndCapture(e->st, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (ce != hipSuccess) return ec_set_hip_error_host(ce, "ec_engine_step: end capture");
        e->graph = g;
        EC_HIP(hipGraphInstantiate(&e->exec, e->graph, nullptr, nullptr, 0));
    }
    EC_HIP(hipGraphLaunch(e->exec, e->st));
    return EC_OK;
}

extern "C" int ec_engine_sync(ec_engine* e) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_sync: null engine");
    EC_HIP(hipStreamSynchronize(e->st));
    return EC_OK;
}

extern "C" int ec_engine_get_tokens(ec_engine* e, int32_t* gen, int32_t* pos) {
    if (!e) return ec_set_error(EC_ERR_ARG, "ec_engine_get_tokens: null engine");
    if (gen) EC_TRY(d2h(e, gen, e->gen, e->B * 4));
    if (pos) EC_TRY(d2h(e, pos, e->pos, e->B * 4));
    return EC_OK;
}

extern "C" int ec_engine_get_logits(ec_engine* e, float* host, uint32_t seq) {
    if (!e || !host || seq >= e->B) return ec_set_error(EC_ERR_ARG, "ec_engine_get_logits: bad argument");
    return d2h(e, host, e->logits + (size_t)seq * e->c.vocab, (size_t)e->c.vocab * 4);
}

extern "C" void* ec_engine_stream(ec_engine* e) { return e ? (void*)e->st : nullptr; }

extern "C" size_t ec_engine_weight_bytes(const ec_engine* e) {
    if (!e) return 0;
    size_t wb = e->weight_bytes + ec_tiled_bytes(e->lm_head.fmt, e->lm_head.N, e->lm_head.K);
    for (const Layer& y : e->L)
        for (const Mat* m : {&y.w_in, &y.w_out, &y.w_gu, &y.w_down}) wb += ec_tiled_bytes(m->fmt, m->N, m->K);
    return wb;
}

// ------------------------------------------------------------ chunked prefill
namespace {
using Lane = ec_engine::PrefillLane;

int prefill_alloc(ec_engine* e, Lane& L, uint32_t i, uint32_t group) {
    if (L.ready) return EC_OK;
    const size_t C = (size_t)group * ec_engine::kPrefillChunk;  // rows of `group` sequences' chunks
    const size_t C1 = ec_engine::kPrefillChunk;                  // per-sequence workspaces
    const size_t wide = std::max({(size_t)e->H, (size_t)e->F, (size_t)e->value_dim, (size_t)e->q_dim});
    // token activations of either matrix format (Q4_K for K % 256 == 0)
    const size_t act_rows_bytes = std::max(ec_gemm_act_bytes(EC_Q8_0, (uint32_t)C, (uint32_t)wide),
                                           ec_gemm_act_bytes(EC_Q4_K, (uint32_t)C, (uint32_t)(wide / 256 * 256)));
    const size_t act1_bytes =
        std::max(ec_act_bytes_pieces(EC_Q8_0, 1, e->H, 2),
                 e->H % 256 ? (size_t)0 : ec_act_bytes_pieces(EC_Q4_K, 1, e->H, 2));
    int rc;
    if (i == 0) {
        L.st = e->st;
    } else if (!L.st) {
        EC_HIP(hipStreamCreateWithFlags(&L.st, hipStreamNonBlocking));
    }
    if ((rc = dalloc(e, &L.x, C * e->H)) || (rc = dalloc(e, &L.n, C * wide)) ||
        (rc = dalloc(e, &L.proj, C * e->nin_max)) || (rc = dalloc(e, &L.gu, C * 2 * (size_t)e->F)) ||
        (rc = dalloc(e, &L.act, L.act_bytes = act_rows_bytes)) || (rc = dalloc(e, &L.act1, act1_bytes)) ||
        (rc = dalloc(e, &L.tok, C)) ||
        (rc = dalloc(e, &L.pos, C)) || (rc = dalloc(e, &L.ctx, C)))
        return rc;
    if (e->value_dim &&
        ((rc = dalloc(e, &L.q, C * e->key_dim)) || (rc = dalloc(e, &L.k, C * e->key_dim)) ||
         (rc = dalloc(e, &L.v, C * e->value_dim)) || (rc = dalloc(e, &L.dec, C * e->n_v)) ||
         (rc = dalloc(e, &L.beta, C * e->n_v)) || (rc = dalloc(e, &L.core, C * e->value_dim)) ||
         (rc = dalloc(e, &L.dnws, ec_deltanet_chunked_ws_bytes((uint32_t)C1, 1, e->n_v)))))
        return rc;
    const size_t aws = ec_attn_prefill_ws_bytes((uint32_t)C1, e->c.n_heads, e->c.max_ctx);
    if (aws && (rc = dalloc(e, &L.aws, aws))) return rc;
    if ((rc = dalloc(e, &L.attn, C * e->q_dim)) ||
        (rc = dalloc(e, &L.ws, ec_attn_ws_bytes(ec_engine::kPrefillAttnSlots, e->c.n_heads, e->c.head_dim,
                                                e->c.max_ctx))))
        return rc;
    L.h_pos.resize(C);
    L.rows = (uint32_t)C;
    L.ready = true;
    return EC_OK;
}

constexpr uint32_t kChunkedDeltaMin = 128;

// y[T][N] (+)= act(x rows) . W  on int8 MFMA (x fp32 [T][K] quantized per
// 32-element block in the matrix's activation format)
int gemm_rows(Lane& L, const Mat& m, const float* x, float* y, uint32_t T, uint32_t ldy, int acc) {
    EC_TRY(ec_gemm_quantize_act(m.fmt, x, L.act, T, m.K, L.st));
    return ec_gemm(m.fmt, m.tiled, L.act, y, T, m.N, m.K, ldy, acc, L.st);
}
// The GEMM on the lane's activation buffer, written by the producing row op.
int gemm_act(Lane& L, const Mat& m, float* y, uint32_t T, uint32_t ldy, int acc) {
    return ec_gemm(m.fmt, m.tiled, L.act, y, T, m.N, m.K, ldy, acc, L.st);
}
// A Q8_0 GEMM's activation is quantized by the row op that produces it (RMSNorm
// rows, SwiGLU rows, gated-norm rows: one launch instead of op + quantize;
// byte-identical); Q4_K matrices and RMSNorm rows wider than 4096 take the fp32
// rows and ec_gemm_quantize_act.
bool fused_act(const Mat& m, uint32_t max_k = 0xFFFFFFFFu) {
    return m.fmt == EC_Q8_0 && m.K % 32 == 0 && (m.K + 127) / 128 * 128 <= max_k;
}
constexpr uint32_t kNormActMaxK = 4096;

// A sequence's chunk inside a prefill pass: T tokens of sequence seq at
// positions p .. p+T-1, in rows r0 .. r0+T-1 of the lane's buffers.
struct PrefillSeg {
    uint32_t seq, T, p, r0;
};

// One pass of the segments' chunks (rows 0 .. M-1, M = the sum of their T,
// L.tok / L.pos already filled) through every block on the lane's stream: the
// row ops and GEMMs take all M rows at once (a ragged multi-sequence GEMM:
// each row's result is the one it gets alone), the ops that read or write a
// sequence's own state (conv ring, recurrent state, KV cache, causal
// attention) run per segment on its rows.
int prefill_chunk(ec_engine* e, Lane& L, const PrefillSeg* sg, uint32_t nsg) {
    const ec_engine_cfg& c = e->c;
    const uint32_t H = e->H, F = e->F;
    hipStream_t st = L.st;
    uint32_t T = 0;  // rows of the pass
    for (uint32_t i = 0; i < nsg; ++i) T += sg[i].T;
    // every launch goes through launch() for ec_engine_prefill_traced (lane 0
    // runs on the engine stream); without a callback it is a plain call
#define EC_PF(op, layer, xin, xout, call) \
    EC_TRY(launch(e, op, layer, 0, xin, xout, [&] { return (call); }))
    EC_PF(EC_OP_PF_EMBED, -1, EC_B_PF_TOK, EC_B_PF_X, ec_glue_embed_fmt(e->embed_fmt, e->embed, L.tok, L.x, T, H, c.vocab, st));
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        Layer& y = e->L[l];
        const int li = (int)l;
        const bool fin = fused_act(y.w_in, kNormActMaxK);
        if (fin)
            EC_PF(EC_OP_PF_NORM, li, EC_B_PF_X, EC_B_PF_ACT,
                  ec_glue_rmsnorm_rows_gemm_act(L.x, y.attn_norm, L.act, T, H, st));
        else
            EC_PF(EC_OP_PF_NORM, li, EC_B_PF_X, EC_B_PF_N, ec_glue_rmsnorm_rows(L.x, y.attn_norm, L.n, T, H, st));
        const int in_buf = fin ? EC_B_PF_ACT : EC_B_PF_N;
        if (!y.attn) {
            const uint32_t Nin = e->nin_delta;
            EC_PF(EC_OP_PF_GEMM_IN, li, in_buf, EC_B_PF_PROJ,
                  fin ? gemm_act(L, y.w_in, L.proj, T, Nin, 0) : gemm_rows(L, y.w_in, L.n, L.proj, T, Nin, 0));
            for (uint32_t i = 0; i < nsg; ++i) {
                const uint32_t s = sg[i].seq, Ts = sg[i].T, p = sg[i].p;
                const size_t r0 = sg[i].r0;
                float* ring = y.conv_state + (size_t)s * c.conv_kernel * e->conv_dim;
                float* state = y.ssm_state + (size_t)s * e->n_v * 128 * 128;
                float *q = L.q + r0 * e->key_dim, *k = L.k + r0 * e->key_dim, *v = L.v + r0 * e->value_dim;
                float *dec = L.dec + r0 * e->n_v, *beta = L.beta + r0 * e->n_v;
                EC_PF(EC_OP_PF_CONV, li, EC_B_PF_PROJ, EC_B_PF_Q,
                      ec_glue_conv_gates_chunk(L.proj + r0 * Nin, Nin, ring, y.conv_w, y.a_log, y.dt_bias, q, k, v,
                                               dec, beta, Ts, p, e->n_k, e->n_v, c.conv_kernel, st));
                // chunked scan from 128 tokens on (MI355X, 32 heads: 64 tokens 21 us
                // token loop vs 29 us chunked; 512 tokens 130 vs 71 us)
                float* core = L.core + r0 * e->value_dim;
                EC_PF(EC_OP_PF_DELTA, li, EC_B_PF_Q, EC_B_PF_CORE,
                      Ts >= kChunkedDeltaMin
                          ? ec_deltanet_chunked(state, q, k, v, dec, beta, core, Ts, 1, e->n_v, e->n_k, 128, 128,
                                                nullptr, L.dnws, st)
                          : ec_deltanet(state, q, k, v, dec, beta, core, Ts, 1, e->n_v, e->n_k, 128, 128, nullptr,
                                        st));
            }
            if (fused_act(y.w_out)) {
                EC_PF(EC_OP_PF_GATED_NORM, li, EC_B_PF_CORE, EC_B_PF_ACT,
                      ec_glue_gated_norm_rows_gemm_act(L.core, L.proj, Nin, e->conv_dim, y.ssm_norm, L.act, T, e->n_v,
                                                       st));
                EC_PF(EC_OP_PF_GEMM_OUT, li, EC_B_PF_ACT, EC_B_PF_X, gemm_act(L, y.w_out, L.x, T, H, 1));
            } else {
                EC_PF(EC_OP_PF_GATED_NORM, li, EC_B_PF_CORE, EC_B_PF_N,
                      ec_glue_gated_norm_rows(L.core, L.proj, Nin, e->conv_dim, y.ssm_norm, L.n, T, e->n_v, st));
                EC_PF(EC_OP_PF_GEMM_OUT, li, EC_B_PF_N, EC_B_PF_X, gemm_rows(L, y.w_out, L.n, L.x, T, H, 1));
            }
        } else {
            const uint32_t Nin = e->nin_attn;
            EC_PF(EC_OP_PF_GEMM_IN, li, in_buf, EC_B_PF_PROJ,
                  fin ? gemm_act(L, y.w_in, L.proj, T, Nin, 0) : gemm_rows(L, y.w_in, L.n, L.proj, T, Nin, 0));
            for (uint32_t i = 0; i < nsg; ++i) {
                const uint32_t s = sg[i].seq, Ts = sg[i].T, p = sg[i].p;
                const size_t r0 = sg[i].r0;
                int8_t* keys = y.keys + (size_t)s * e->seq_stride;
                int8_t* vals = y.vals + (size_t)s * e->seq_stride;
                float* ks = y.ks + (size_t)s * e->ctx_stride * c.n_kv;
                float* vs = y.vs + (size_t)s * e->ctx_stride * c.n_kv;
                float* qn = L.n + r0 * e->q_dim;
                float* ao = L.attn + r0 * e->q_dim;
                int32_t* cx = L.ctx + r0;
                // slots = the chunk's tokens sharing sequence s's cache (seq_stride 0)
                EC_PF(EC_OP_PF_ROPE_APPEND, li, EC_B_PF_PROJ, EC_B_PF_N,
                      ec_glue_qk_rope_append(L.proj + r0 * Nin, Nin, y.q_norm, y.k_norm, y.use_qn, y.use_kn,
                                             e->inv_freq, L.pos + r0, qn, nullptr, nullptr, keys, vals, ks, vs, cx,
                                             Ts, 0, c.max_ctx, c.n_heads, c.n_kv, c.head_dim, st));
                // causal attention of the chunk's T queries (positions p .. p+T-1)
                // over the sequence's cache, one pass per 32/G query tokens
                const uint32_t G = c.n_heads / c.n_kv;
                EC_PF(EC_OP_PF_ATTN, li, EC_B_PF_N, EC_B_PF_ATTN, [&]() -> int {
                    if (G == 1 || G == 2 || G == 4)
                        return ec_attn_prefill(qn, keys, vals, ks, vs, ao, Ts, (int32_t)p, c.n_heads, c.n_kv,
                                               c.head_dim, c.max_ctx, L.aws, st);
                    // other group sizes: the decode kernel with the chunk's tokens
                    // as slots sharing the cache (ctx = position + 1)
                    for (uint32_t s0 = 0; s0 < Ts; s0 += ec_engine::kPrefillAttnSlots) {
                        const uint32_t n = std::min(Ts - s0, ec_engine::kPrefillAttnSlots);
                        EC_TRY(ec_attn_decode(qn + (size_t)s0 * e->q_dim, keys, vals, ks, vs,
                                              ao + (size_t)s0 * e->q_dim, cx + s0, n, 0, c.n_heads, c.n_kv,
                                              c.head_dim, c.max_ctx, L.ws, st));
                    }
                    return EC_OK;
                }());
            }
            EC_PF(EC_OP_PF_GEMM_OUT, li, EC_B_PF_ATTN, EC_B_PF_X, gemm_rows(L, y.w_out, L.attn, L.x, T, H, 1));
        }
        if (fused_act(y.w_gu, kNormActMaxK)) {
            EC_PF(EC_OP_PF_NORM, li, EC_B_PF_X, EC_B_PF_ACT,
                  ec_glue_rmsnorm_rows_gemm_act(L.x, y.ffn_norm, L.act, T, H, st));
            EC_PF(EC_OP_PF_GEMM_GU, li, EC_B_PF_ACT, EC_B_PF_GU, gemm_act(L, y.w_gu, L.gu, T, 2 * F, 0));
        } else {
            EC_PF(EC_OP_PF_NORM, li, EC_B_PF_X, EC_B_PF_N, ec_glue_rmsnorm_rows(L.x, y.ffn_norm, L.n, T, H, st));
            EC_PF(EC_OP_PF_GEMM_GU, li, EC_B_PF_N, EC_B_PF_GU, gemm_rows(L, y.w_gu, L.n, L.gu, T, 2 * F, 0));
        }
        if (fused_act(y.w_down)) {
            EC_PF(EC_OP_PF_SWIGLU, li, EC_B_PF_GU, EC_B_PF_ACT, ec_glue_swiglu_rows_gemm_act(L.gu, L.act, T, F, st));
            EC_PF(EC_OP_PF_GEMM_DOWN, li, EC_B_PF_ACT, EC_B_PF_X, gemm_act(L, y.w_down, L.x, T, H, 1));
        } else {
            EC_PF(EC_OP_PF_SWIGLU, li, EC_B_PF_GU, EC_B_PF_N, ec_glue_swiglu_rows(L.gu, L.n, T, F, st));
            EC_PF(EC_OP_PF_GEMM_DOWN, li, EC_B_PF_N, EC_B_PF_X, gemm_rows(L, y.w_down, L.n, L.x, T, H, 1));
        }
    }
#undef EC_PF
    return EC_OK;
}

// Prefill job of one sequence on a lane: the next chunk to run.
struct PrefillJob {
    uint32_t seq, n;
    const int32_t* tokens;
    int32_t pos0;
    uint32_t done = 0;  // tokens already enqueued
};

// The last token's logits and greedy next token of a finished job, whose last
// chunk sits in the lane's rows r0 .. r0+T-1; pos[seq] = pos0 + n.
int prefill_head(ec_engine* e, Lane& L, const PrefillJob& j, uint32_t r_last) {
    const int32_t last = j.pos0 + (int32_t)j.n - 1;
    const float* xl = L.x + (size_t)r_last * e->H;
    EC_TRY(launch(e, EC_OP_PF_HEAD, -1, 0, EC_B_PF_X, EC_B_LOGITS, [&]() -> int {
        if (e->lm_head.fmt == EC_Q4_K) {
            EC_TRY(ec_glue_rmsnorm_rows(xl, e->final_norm, L.n, 1, e->H, L.st));
            EC_TRY(ec_quantize_act_pieces(EC_Q4_K, L.n, L.act1, 1, e->H, e->P, L.st));
        } else {
            EC_TRY(ec_glue_rmsnorm_quant_pieces(xl, e->final_norm, L.act1, 1, e->H, e->P, L.st));
        }
        return ec_matvec_pieces(e->lm_head.fmt, e->P, e->lm_head.tiled, L.act1,
                                e->logits + (size_t)j.seq * e->c.vocab, 1, e->c.vocab, e->H, e->c.vocab, 0, L.st);
    }));
    EC_HIP(hipMemcpyAsync(e->pos + j.seq, &last, 4, hipMemcpyHostToDevice, L.st));
    EC_TRY(ec_glue_argmax_advance_bounded(e->logits + (size_t)j.seq * e->c.vocab, e->c.vocab, e->gen + j.seq,
                                          e->tok + j.seq, e->pos + j.seq, 1, e->c.max_ctx, L.st));
    EC_HIP(hipStreamSynchronize(L.st));  // `last` lives on this frame
    return EC_OK;
}

// Enqueue the next chunk of each of the lane's jobs (at most its row
// capacity / kPrefillChunk) as one pass, job i's chunk after job i-1's rows
// (the lane's previous pass must have completed: its token / position rows
// are overwritten).
int prefill_step(ec_engine* e, Lane& L, PrefillJob* const* js, uint32_t nj) {
    const uint32_t C = ec_engine::kPrefillChunk;
    PrefillSeg sg[ec_engine::kPrefillGroup];
    uint32_t r0 = 0;
    for (uint32_t i = 0; i < nj; ++i) {
        const PrefillJob& j = *js[i];
        const uint32_t T = std::min(j.n - j.done, C), p = (uint32_t)j.pos0 + j.done;
        for (uint32_t t = 0; t < T; ++t) L.h_pos[r0 + t] = (int32_t)(p + t);
        EC_HIP(hipMemcpyAsync(L.tok + r0, j.tokens + j.done, T * 4, hipMemcpyHostToDevice, L.st));
        sg[i] = {j.seq, T, p, r0};
        r0 += T;
    }
    EC_HIP(hipMemcpyAsync(L.pos, L.h_pos.data(), r0 * 4, hipMemcpyHostToDevice, L.st));
    EC_HIP(hipStreamSynchronize(L.st));  // pageable sources: the copies are complete before h_pos is reused
    EC_TRY(prefill_chunk(e, L, sg, nj));
    for (uint32_t i = 0; i < nj; ++i) {
        PrefillJob& j = *js[i];
        j.done += sg[i].T;
        if (j.done == j.n) EC_TRY(prefill_head(e, L, j, sg[i].r0 + sg[i].T - 1));
    }
    return EC_OK;
}

// Run the jobs over `lanes` lanes of `group` sequences each: a lane's slots
// take the next unstarted job when theirs is done, and each pass runs one
// chunk of every job the lane holds; lanes alternate so that one lane's pass
// is queued while another's runs.
int prefill_run(ec_engine* e, std::vector<PrefillJob>& jobs, uint32_t lanes, uint32_t group) {
    group = std::max(1u, std::min(group, ec_engine::kPrefillGroup));
    lanes = std::max(1u, std::min({lanes, ec_engine::kPrefillLanes,
                                   (uint32_t)((jobs.size() + group - 1) / group)}));
    for (uint32_t i = 0; i < lanes; ++i) EC_TRY(prefill_alloc(e, e->pf[i], i, group));
    for (uint32_t i = 0; i < lanes; ++i)  // lanes allocated earlier may hold fewer rows
        group = std::min(group, e->pf[i].rows / ec_engine::kPrefillChunk);
    EC_HIP(hipStreamSynchronize(e->st));  // whatever the decode stream queued before
    std::vector<int> cur((size_t)lanes * group, -1);
    uint32_t next = 0;
    int rc = EC_OK;
    for (bool any = true; any && rc == EC_OK;) {
        any = false;
        for (uint32_t i = 0; i < lanes && rc == EC_OK; ++i) {
            PrefillJob* act[ec_engine::kPrefillGroup];
            uint32_t na = 0;
            for (uint32_t g = 0; g < group; ++g) {
                int& c = cur[(size_t)i * group + g];
                if (c < 0 || jobs[c].done == jobs[c].n) c = next < jobs.size() ? (int)next++ : -1;
                if (c >= 0) act[na++] = &jobs[c];
            }
            if (na == 0) continue;
            any = true;
            rc = prefill_step(e, e->pf[i], act, na);
        }
    }
    // every lane drained, also after an error (no work left in flight)
    for (uint32_t i = 0; i < lanes; ++i) {
        const hipError_t se = hipStreamSynchronize(e->pf[i].st);
        if (rc == EC_OK && se != hipSuccess) rc = ec_set_hip_error_host(se, "ec_engine_prefill: stream");
    }
    return rc;
}

// Sequences per prefill pass (EC_PREFILL_GROUP = 1 .. 4, for comparison).
uint32_t prefill_group() {
    static const uint32_t g = [] {
        const char* v = getenv("EC_PREFILL_GROUP");
        const uint32_t n = v ? (uint32_t)atoi(v) : 0u;
        return n >= 1 && n <= ec_engine::kPrefillGroup ? n : 2u;
    }();
    return g;
}

int check_prefill_args(ec_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n, int32_t pos0, const char* who) {
    if (!e || !tokens || n == 0 || seq >= e->B || pos0 < 0 || (uint64_t)pos0 + n > e->c.max_ctx) {
        char buf[160];
        snprintf(buf, sizeof buf, "%s: bad argument (seq < max_batch, pos0 + n <= max_ctx)", who);
        return ec_set_error(EC_ERR_ARG, buf);
    }
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= e->c.vocab) {
            char buf[96];
            snprintf(buf, sizeof buf, "%s: token id", who);
            return ec_set_error(EC_ERR_ARG, buf);
        }
    if (e->c.head_dim != 256) return ec_set_error(EC_ERR_UNSUPPORTED, "ec_engine_prefill: head_dim must be 256");
    return EC_OK;
}
}  // namespace

extern "C" int ec_engine_prefill(ec_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n, int32_t pos0) {
    EC_TRY(check_prefill_args(e, seq, tokens, n, pos0, "ec_engine_prefill"));
    std::vector<PrefillJob> jobs{PrefillJob{seq, n, tokens, pos0}};
    return prefill_run(e, jobs, 1, prefill_group());
}

extern "C" int ec_engine_prefill_traced(ec_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n, int32_t pos0,
                                        ec_trace_fn cb, void* user) {
    EC_TRY(check_prefill_args(e, seq, tokens, n, pos0, "ec_engine_prefill_traced"));
    if (!cb) return ec_set_error(EC_ERR_ARG, "ec_engine_prefill_traced: null callback");
    std::vector<PrefillJob> jobs{PrefillJob{seq, n, tokens, pos0}};
    e->trace_cb = cb;
    e->trace_user = user;
    const int rc = prefill_run(e, jobs, 1, prefill_group());
    e->trace_cb = nullptr;
    e->trace_user = nullptr;
    return rc;
}

extern "C" int ec_engine_prefill_batch(ec_engine* e, uint32_t n_seqs, const uint32_t* seqs,
                                       const int32_t* const* tokens, const uint32_t* lens, const int32_t* pos0) {
    if (!e || !seqs || !tokens || !lens || !pos0) return ec_set_error(EC_ERR_ARG, "ec_engine_prefill_batch: null argument");
    std::vector<PrefillJob> jobs;
    for (uint32_t i = 0; i < n_seqs; ++i) {
        EC_TRY(check_prefill_args(e, seqs[i], tokens[i], lens[i], pos0[i], "ec_engine_prefill_batch"));
        for (uint32_t k = 0; k < i; ++k)
            if (seqs[k] == seqs[i]) return ec_set_error(EC_ERR_ARG, "ec_engine_prefill_batch: a sequence appears twice");
        jobs.push_back(PrefillJob{seqs[i], lens[i], tokens[i], pos0[i]});
    }
    if (jobs.empty()) return EC_OK;
    // Two lanes of two sequences each (the 4B benchmark's eight prompts on one
    // box, tok/s, lanes x sequences per pass: 4 x 1 48.3k, 2 x 2 49.0k, 3 x 2
    // 48.7k, 4 x 2 48.6k, 2 x 4 48.2k, 1 x 4 46.3k; one lane of one sequence
    // 37.8k).  EC_PREFILL_LANES = 1 .. 4 sets the lanes, for comparison.
    static const uint32_t lanes_env = [] {
        const char* v = getenv("EC_PREFILL_LANES");
        return v ? (uint32_t)atoi(v) : 0u;
    }();
    return prefill_run(e, jobs, lanes_env >= 1 ? lanes_env : 2u, prefill_group());
}

extern "C" int ec_engine_profile_matvecs(ec_engine* e, uint32_t reps, uint32_t* launches, double* bytes_per_step,
                                         double* us_per_step) {
    if (!e || !launches || !bytes_per_step || !us_per_step || reps == 0)
        return ec_set_error(EC_ERR_ARG, "ec_engine_profile_matvecs: bad argument");
    std::vector<double> by;
    hipGraph_t g = nullptr;
    hipGraphExec_t x = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    EC_HIP(hipStreamSynchronize(e->st));
    EC_HIP(hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
    e->mv_only = true;
    e->mv_bytes = &by;
    int rc = record_step(e);
    e->mv_only = false;
    e->mv_bytes = nullptr;
    const hipError_t ce = hipStreamEndCapture(e->st, &g);
    if (!rc && ce != hipSuccess) rc = ec_set_hip_error_host(ce, "ec_engine_profile_matvecs: capture");
    auto run = [&]() -> int {
        EC_HIP(hipGraphInstantiate(&x, g, nullptr, nullptr, 0));
        EC_HIP(hipGraphLaunch(x, e->st));  // warm-up replay
        EC_HIP(hipEventCreate(&a));
        EC_HIP(hipEventCreate(&b));
        EC_HIP(hipEventRecord(a, e->st));
        for (uint32_t r = 0; r < reps; ++r) EC_HIP(hipGraphLaunch(x, e->st));
        EC_HIP(hipEventRecord(b, e->st));
        EC_HIP(hipEventSynchronize(b));
        float ms = 0.0f;
        EC_HIP(hipEventElapsedTime(&ms, a, b));
        *us_per_step = ms * 1e3 / reps;
        return EC_OK;
    };
    if (!rc) rc = run();
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (x) (void)hipGraphExecDestroy(x);
    if (g) (void)hipGraphDestroy(g);
    *launches = (uint32_t)by.size();
    double t = 0.0;
    for (double v : by) t += v;
    *bytes_per_step = t;
    return rc;
}

extern "C" int ec_engine_step_traced(ec_engine* e, ec_trace_fn cb, void* user) {
    if (!e || !cb) return ec_set_error(EC_ERR_ARG, "ec_engine_step_traced: null argument");
    e->trace_cb = cb;
    e->trace_user = user;
    const int rc = record_step(e);
    e->trace_cb = nullptr;
    e->trace_user = nullptr;
    return rc;
}

extern "C" int ec_engine_buffer(ec_engine* e, int which, void** dev, size_t* bytes) {
    if (!e || !dev || !bytes) return ec_set_error(EC_ERR_ARG, "ec_engine_buffer: null argument");
    const ec_engine_cfg& c = e->c;
    const size_t B = e->B;
    void* p = nullptr;
    size_t n = 0;
    switch (which) {
        case EC_B_X: p = e->x, n = B * e->H * 4; break;
        case EC_B_X2: p = e->x2, n = B * e->H * 4; break;
        case EC_B_PARTS: p = e->parts, n = (size_t)kMaxResidSplit * B * e->H * 4; break;
        case EC_B_PROJ: p = e->proj, n = (size_t)kMaxResidSplit * B * e->nin_max * 4; break;
        case EC_B_GU: p = e->gu, n = (size_t)kMaxResidSplit * B * 2 * e->F * 4; break;
        case EC_B_ACT_H: p = e->act_h, n = ec_act_bytes_pieces(EC_Q8_0, e->B, e->H, e->P); break;
        case EC_B_ACT_V: p = e->act_v, n = ec_act_bytes_pieces(EC_Q8_0, e->B, e->value_dim, e->P); break;
        case EC_B_ACT_F: p = e->act_f, n = ec_act_bytes_pieces(EC_Q8_0, e->B, e->F, e->P); break;
        case EC_B_ACT_Q: p = e->act_q, n = ec_act_bytes_pieces(EC_Q8_0, e->B, e->q_dim, e->P); break;
        case EC_B_ATTN_OUT: p = e->attn_out, n = B * e->q_dim * 4; break;
        case EC_B_Q_PACKED: p = e->q_packed, n = e->q_packed ? ec_attn_qa_bytes(e->B, c.n_heads) : 0; break;
        case EC_B_Q_SCALES: p = e->q_scales, n = e->q_scales ? B * c.n_heads * 3 * 4 : 0; break;
        case EC_B_QBUF: p = e->qbuf, n = B * e->q_dim * 4; break;
        case EC_B_LOGITS: p = e->logits, n = B * c.vocab * 4; break;
        case EC_B_TOK: p = e->tok, n = B * 4; break;
        case EC_B_POS: p = e->pos, n = B * 4; break;
        case EC_B_GEN: p = e->gen, n = B * 4; break;
        case EC_B_CTX: p = e->ctx, n = B * 4; break;
        case EC_B_INV_FREQ: p = e->inv_freq, n = (size_t)c.head_dim / 2 * 4; break;
        case EC_B_HN: p = e->hn, n = e->hn ? B * e->H * 4 : 0; break;
        case EC_B_CORE: p = e->core_f, n = e->core_f ? B * e->value_dim * 4 : 0; break;
        case EC_B_FF: p = e->ff, n = e->ff ? B * e->F * 4 : 0; break;
        case EC_B_ACT4_H: p = e->act4_h, n = e->q4 ? ec_act_bytes_pieces(EC_Q4_K, e->B, e->H, e->P) : 0; break;
        case EC_B_ACT4_V:
            p = e->act4_v, n = e->q4 && e->value_dim % 256 == 0 ? ec_act_bytes_pieces(EC_Q4_K, e->B, e->value_dim, e->P) : 0;
            break;
        case EC_B_ACT4_Q: p = e->act4_q, n = e->q4 ? ec_act_bytes_pieces(EC_Q4_K, e->B, e->q_dim, e->P) : 0; break;
        case EC_B_ACT4_F: p = e->act4_f, n = e->q4 && e->F % 256 == 0 ? ec_act_bytes_pieces(EC_Q4_K, e->B, e->F, e->P) : 0; break;
        default: {
            // chunk buffers of prefill lane 0 (none before the first prefill)
            const ec_engine::PrefillLane& L = e->pf[0];
            const size_t C = ec_engine::kPrefillChunk * 4;
            const size_t wide = std::max({(size_t)e->H, (size_t)e->F, (size_t)e->value_dim, (size_t)e->q_dim});
            const bool r = L.ready, d = r && e->value_dim;
            switch (which) {
                case EC_B_PF_X: p = L.x, n = r ? C * e->H : 0; break;
                case EC_B_PF_N: p = L.n, n = r ? C * wide : 0; break;
                case EC_B_PF_PROJ: p = L.proj, n = r ? C * e->nin_max : 0; break;
                case EC_B_PF_Q: p = L.q, n = d ? C * e->key_dim : 0; break;
                case EC_B_PF_K: p = L.k, n = d ? C * e->key_dim : 0; break;
                case EC_B_PF_V: p = L.v, n = d ? C * e->value_dim : 0; break;
                case EC_B_PF_DEC: p = L.dec, n = d ? C * e->n_v : 0; break;
                case EC_B_PF_BETA: p = L.beta, n = d ? C * e->n_v : 0; break;
                case EC_B_PF_CORE: p = L.core, n = d ? C * e->value_dim : 0; break;
                case EC_B_PF_GU: p = L.gu, n = r ? C * 2 * e->F : 0; break;
                case EC_B_PF_ATTN: p = L.attn, n = r ? C * e->q_dim : 0; break;
                case EC_B_PF_TOK: p = L.tok, n = r ? C : 0; break;
                case EC_B_PF_ACT1:
                    p = L.act1, n = r ? ec_act_bytes_pieces(e->lm_head.fmt == EC_Q4_K ? EC_Q4_K : EC_Q8_0, 1, e->H, e->P) : 0;
                    break;
                case EC_B_PF_ACT: p = L.act, n = r ? L.act_bytes : 0; break;
                default: return ec_set_error(EC_ERR_ARG, "ec_engine_buffer: unknown buffer");
            }
            if (!r) p = nullptr;
        }
    }
    *dev = p;
    *bytes = n;
    return EC_OK;
}
