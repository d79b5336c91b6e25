// Uses every function and member function declared by the reference-signature
// headers, so that `nm -u` of this object lists the mangled symbols a program
// built against those headers needs from libechohip.so.  Compiled, never run.
#include "kernels/matvec.h"
#include "kernels/quant.h"
#include "kv_cache.h"

void abi_use(const ModelConfig& cfg, void* p, float* f, int8_t* q, uint16_t* h) {
    quantize_per_token_symmetric(f, q, f, 1, 1);
    fused_dequant_dot_int8(f, q, f, f, 1, 1);
    (void)fused_dequant_dot_q8_0((const block_q8_0*)p, 1, f);
    (void)fused_dequant_dot_q4_K((const block_q4_K*)p, 1, f);
    dequantize_q8_0_to_fp16(p, h, 32);
    dequantize_q4_K_to_fp16(p, h, 256);
    dequantize_q2_K_to_fp16(p, h, 256);
    matvec_fp16_fp32<1024, 512>(h, f, f, 1, 1);
    matvec_fp16_fp32<2048, 1024>(h, f, f, 1, 1);
    matvec_dispatch(h, f, f, 1, 1, cfg);
    matvec_q8_0(p, f, f, 1, 32);
    matvec_q4_K(p, f, f, 1, 256);
    matvec_q2_K(p, f, f, 1, 256);
    KVCache kv(cfg);
    const KVCache& ckv = kv;
    kv.append(0, f, f);
    (void)kv.layer(0);
    (void)ckv.layer(0);
    (void)kv.seq_len();
    kv.reset();
}
