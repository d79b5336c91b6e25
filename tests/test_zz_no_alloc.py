"""ec_attn_decode_noalloc (include/echo_hip.h): attention decode with the
library's fixed per-GPU scratch instead of a caller workspace, for callers
that cannot allocate.  Checked against ec_attn_decode with its own workspace
(same kernels: bit-identical outputs) on two calls in a row, the second with
a smaller input (fewer sequences, shorter contexts), so the scratch keeps the
first call's contents when the second runs; a workspace larger than the
scratch is refused before any launch."""
import numpy as np
import pytest

from test_gpu_kernels import _kv_case, dev, empty, host

pytestmark = pytest.mark.gpu


def _call_both(hip, oc, ctxs, max_ctx, n_heads, n_kv, hd, seed):
    import torch
    n_seq = len(ctxs)
    keys, vals, ks, vs, _, _ = _kv_case(oc, n_seq, ctxs, max_ctx, n_kv, hd, seed)
    q = np.random.default_rng(seed).standard_normal((n_seq, n_heads * hd)).astype(np.float32)
    args = (dev(q), dev(keys), dev(vals), dev(ks), dev(vs))
    ctx = dev(np.array(ctxs, np.int32))
    stride = max_ctx * n_kv * hd
    a = empty(n_seq * n_heads * hd, torch.float32)
    ws = empty(hip.attn_ws_bytes(n_seq, n_heads, hd, max_ctx), torch.uint8)
    hip.attn_decode(*args, a, ctx, n_seq, stride, n_heads, n_kv, hd, max_ctx, ws)
    b = empty(n_seq * n_heads * hd, torch.float32)
    hip.attn_decode_noalloc(*args, b, ctx, n_seq, stride, n_heads, n_kv, hd, max_ctx)
    torch.cuda.synchronize()
    return host(a), host(b)


def test_noalloc_attention_matches_workspace_entry_point(hip, oc):
    print("noalloc: large call (4 sequences, ctx up to 3000, GQA 16/4)", flush=True)
    a, b = _call_both(hip, oc, [3000, 1, 777, 64], 3072, 16, 4, 256, 91)
    assert np.array_equal(a, b)
    print("noalloc: smaller second call (1 sequence, ctx 100)", flush=True)
    a, b = _call_both(hip, oc, [100], 128, 16, 4, 256, 92)
    assert np.array_equal(a, b)
    print("noalloc: fp32 attention path (head_dim 128)", flush=True)
    a, b = _call_both(hip, oc, [200, 5], 256, 8, 2, 128, 93)
    assert np.array_equal(a, b)


def test_noalloc_attention_rejects_oversized_workspace(hip):
    from echohip.lib import EchoHipError
    cap = hip.attn_noalloc_max_bytes()
    assert cap == 16 << 20
    max_ctx = 1 << 20  # 16 heads x 16384 chunks of 64 positions x 1040 B > 16 MiB
    assert hip.attn_ws_bytes(1, 16, 256, max_ctx) > cap
    import torch
    buf = empty(4096, torch.float32)  # real (small) buffers: the size check refuses the call before any launch
    ctx = dev(np.array([1], np.int32))
    with pytest.raises(EchoHipError, match="exceeds the fixed"):
        hip.attn_decode_noalloc(buf, buf, buf, buf, buf, buf, ctx, 1, 0, 16, 4, 256, max_ctx)
