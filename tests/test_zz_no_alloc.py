"""k3x_moe_prefill_noalloc (the prefill path with its working buffers in a static device
array) against k3x_moe_forward, the entry point it is a variant of, on two calls in a row,
the second with fewer tokens (the array keeps the first call's contents), at the tiny
shape and at the full K2 shape: the same routing bit for bit, and the same outputs bit for
bit with fp32 input, within 1e-6 relative with bf16 input (where k3x_moe_forward hands the
shared expert's products to hipBLASLt, which the no-allocation path does not call); sizes
beyond the array, and decode-sized calls, refused with K3X_E_SHAPE."""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, say, synth_layer

pytestmark = pytest.mark.gpu


def both(torch, k3x, layer, x, bf16):
    T, H = x.shape
    K = layer.cfg.topk
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    if bf16:
        xt = xt.to(torch.bfloat16)
    dt = k3x.K3X_BF16 if bf16 else k3x.K3X_F32
    r = torch.from_numpy(np.ascontiguousarray(x[:, ::-1])).cuda().float().contiguous()
    outs = []
    s = torch.cuda.current_stream().cuda_stream
    for fn in (layer.forward, layer.prefill_noalloc):
        out = torch.full((T, H), 3.0, dtype=torch.float32, device="cuda")
        idx = torch.full((T, K), -7, dtype=torch.int32, device="cuda")
        wt = torch.zeros((T, K), dtype=torch.float32, device="cuda")
        fn(out.data_ptr(), xt.data_ptr(), T, dt, r.data_ptr(), idx.data_ptr(), wt.data_ptr(),
           stream=s)
        torch.cuda.synchronize()
        outs.append((out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()))
    layer.check()
    return outs


def test_noalloc_tiny_two_calls(torch, k3x):
    say("case: no-alloc prefill, tiny layer, T=300 then T=40, vs k3x_moe_forward")
    L = synth.tiny(seed=41)
    layer = bank_layer(k3x, L)
    for T, bf16 in ((300, False), (40, True)):
        x = L.x(T, bf16=bf16, stream_sub=200 + T)
        (o1, i1, w1), (o2, i2, w2) = both(torch, k3x, layer, x, bf16)
        say(f"  T={T}: equal={np.array_equal(o1, o2)} rel_l2={synth.rel_l2(o2, o1):.2e}")
        assert np.array_equal(i1, i2) and np.array_equal(w1, w2)
        assert synth.rel_l2(o2, o1) < 1e-6 if bf16 else np.array_equal(o1, o2)
        o, ri, _, _ = L.oracle_moe(x)
        assert np.array_equal(i2, ri)
        assert synth.rel_l2(o2 - x[:, ::-1], o) < 1e-3
    xd = torch.zeros((5000, L.H), dtype=torch.float32, device="cuda")
    with pytest.raises(k3x.K3XError) as ei:
        layer.prefill_noalloc(xd.data_ptr(), xd.data_ptr(), 5000)
    assert ei.value.status == -2
    with pytest.raises(k3x.K3XError) as ei:
        layer.prefill_noalloc(xd.data_ptr(), xd.data_ptr(), 8)
    assert ei.value.status == -2
    layer.close()


def test_noalloc_full_shape(torch, k3x):
    say("case: no-alloc prefill, full K2 layer, T=111 then T=24, T=112 refused")
    L = synth.full(seed=42, zipf_alpha=1.0)
    layer = synth_layer(k3x, L)
    for T in (111, 24):
        x = L.x(T, bf16=True, stream_sub=300 + T)
        (o1, i1, w1), (o2, i2, w2) = both(torch, k3x, layer, x, True)
        say(f"  T={T}: equal={np.array_equal(o1, o2)} rel_l2={synth.rel_l2(o2, o1):.2e}")
        assert np.array_equal(i1, i2) and np.array_equal(w1, w2)
        assert synth.rel_l2(o2, o1) < 1e-6
    xd = torch.zeros((112, L.H), dtype=torch.float32, device="cuda")
    with pytest.raises(k3x.K3XError) as ei:
        layer.prefill_noalloc(xd.data_ptr(), xd.data_ptr(), 112)
    assert ei.value.status == -2
    layer.close()
