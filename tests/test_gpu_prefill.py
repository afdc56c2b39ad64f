"""GPU parity of the prefill pipeline (more than 8 tokens per call), through the C ABI.

Same bar as the decode path: selected expert indices bit-exact (ties to the lower index),
routing weights to float rounding, outputs within TOL relative L2 of the oracle, which is
bitwise the reference's k3_moe / k3_moe_prefill.  At the full size (2048 tokens, Zipf-
skewed routing) every token is checked against the oracle's router, the whole layer on
the host (the compiled reference's prefill, pinned bitwise to the oracle) and the
decode path, whose grouping of tokens must not change any result.
"""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, host_layer, per_token_rel, say, synth_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3          # relative L2, the parity bar


def decode_forward(torch, k3x, layer, x, bf16):
    """The same tokens through the decode path, 8 at a time."""
    outs, idxs, wts = [], [], []
    for t0 in range(0, x.shape[0], 8):
        o, i, w = dev_forward(torch, k3x, layer, x[t0:t0 + 8], bf16=bf16)
        outs.append(o); idxs.append(i); wts.append(w)
    return np.concatenate(outs), np.concatenate(idxs), np.concatenate(wts)


@pytest.mark.parametrize("T,bf16", [(9, False), (37, False), (37, True), (130, True)])
def test_tiny_prefill_vs_oracle(torch, k3x, T, bf16):
    say(f"case: tiny layer prefill T={T} bf16={bf16} vs oracle")
    L = synth.tiny(seed=11)
    layer = bank_layer(k3x, L)
    x = L.x(T, bf16=bf16, stream_sub=T)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=bf16)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    layer.close()


def test_tiny_prefill_special_scales_and_resid(torch, k3x):
    """Scale bytes 255 (group zeroed) and a wide exponent range take the exact
    dequantisation kernels; resid + MoE."""
    say("case: tiny layer prefill, scale bytes 255 and 100..140, with residual")
    L = synth.tiny(seed=12, scale_lo=100, scale_hi=140)
    for e in range(L.E):
        d = L.expert(e)
        d["s1"][0, 1] = 255
        d["s3"][5, 0] = 255
        d["s2"][7, 2] = 255
    layer = bank_layer(k3x, L)
    x = L.x(40, bf16=False)
    r = L.x(40, bf16=False, stream_sub=77)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x, resid=r)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o + r)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    layer.close()


def test_tiny_prefill_grouping_invariant(torch, k3x):
    """Prefill of 64 tokens equals the decode path over the same tokens 8 at a time."""
    say("case: tiny layer, prefill T=64 vs decode in groups of 8")
    L = synth.tiny(seed=13)
    layer = bank_layer(k3x, L)
    x = L.x(64, bf16=False, stream_sub=3)
    out, idx, wt = dev_forward(torch, k3x, layer, x)
    o2, i2, w2 = decode_forward(torch, k3x, layer, x, False)
    assert np.array_equal(idx, i2)
    np.testing.assert_allclose(wt, w2, rtol=1e-6)
    err = synth.rel_l2(out, o2)
    say(f"  rel_l2(prefill, decode)={err:.3e}")
    assert err < 1e-5
    layer.close()


def test_full_prefill_2048_zipf(torch, k3x):
    """The full-size layer, one 2048-token chunk of bf16 activations, Zipf-skewed bias:
    the routing of every token against the oracle's router, and every token against the
    decode path and against the whole layer on the host (the reference's prefill;
    t_moe_prefill holds a whole chunk bitwise, test_ops.c:891-1014), each within TOL."""
    import oracle_lib as ol
    say("case: full-size prefill, 2048 bf16 tokens, Zipf bias (alpha 1.0, s 1.1)")
    L = synth.full(seed=3, zipf_alpha=1.0)
    layer = synth_layer(k3x, L)
    T = 2048
    x = L.x(T, bf16=True, stream_sub=5)
    out, idx, wt = dev_forward(torch, k3x, layer, x, bf16=True)
    counts = np.bincount(idx.ravel(), minlength=L.E)
    say(f"  experts used {int((counts > 0).sum())}, tokens per expert max {counts.max()} "
        f"median {int(np.median(counts))}")
    # routing of every token against the oracle's router (the reference's arithmetic)
    ri = np.empty((T, L.K), np.int32)
    rw = np.empty((T, L.K), np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_router(ol.ptr(ri[t], ol.I32P), ol.ptr(rw[t], ol.F32P),
                              ol.ptr(xt, ol.F32P), ol.ptr(L.gate, ol.F32P),
                              ol.ptr(L.bias, ol.F32P), L.H, L.E, L.K, 1, 2.5)
    assert np.array_equal(idx, ri)
    np.testing.assert_allclose(wt, rw, rtol=1e-6)
    say("  routing of all 2048 tokens equals the oracle's")
    # every token against the decode path
    o2, i2, _ = decode_forward(torch, k3x, layer, x, True)
    assert np.array_equal(idx, i2)
    err = synth.rel_l2(out, o2)
    say(f"  rel_l2(prefill, decode) over 2048 tokens = {err:.3e}")
    assert err < 1e-5
    # every token against the whole layer on the host, token by token
    o, what = host_layer(L, x, ri)
    r = per_token_rel(out, o)
    say(f"  {T} tokens against {what}: per-token rel_l2 median {np.median(r):.2e} "
        f"max {r.max():.2e}")
    assert r.max() < TOL
    layer.close()


@pytest.mark.parametrize("latent,bf16", [(False, False), (False, True), (True, True)])
def test_prefill_graph_replays(torch, k3x, latent, bf16):
    """A prefill chunk (T = 40) captured once into a HIP graph and replayed on new inputs,
    with eager work and synchronisations between the replays: every replay equals the eager
    call bit for bit (routing, permute, grouped GEMMs and combine are all kernels with
    host-computed grids, so the per-layer sequence captures).  bf16 input takes the shared
    expert's library GEMMs (and in the latent form the projections' library GEMMs) into
    the graph; fp32 input the dense kernel."""
    say(f"case: prefill T=40 captured in a graph, 3 replays with eager copies between, "
        f"latent={latent} bf16={bf16}")
    L = synth.tiny_latent(seed=35) if latent else synth.tiny(seed=35)
    layer = bank_layer(k3x, L)
    T, H, K = 40, L.H, L.K
    xd = torch.empty((T, H), dtype=torch.bfloat16 if bf16 else torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((T, K), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()

    def run():
        layer.forward(out.data_ptr(), xd.data_ptr(), T, k3x.K3X_BF16 if bf16 else k3x.K3X_F32,
                      0, idx.data_ptr(), wt.data_ptr(), stream=s.cuda_stream)

    xd.copy_(torch.from_numpy(L.x(T, bf16=bf16, stream_sub=20)))
    with torch.cuda.stream(s):
        run()                                   # eager: reserves the chunk buffers
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.synchronize()
    for r in range(3):
        x = L.x(T, bf16=bf16, stream_sub=21 + r)
        xd.copy_(torch.from_numpy(x))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        go, gi = out.clone(), idx.clone()
        with torch.cuda.stream(s):
            run()
        torch.cuda.synchronize()
        say(f"  replay {r}")
        assert torch.equal(gi, idx) and torch.equal(go, out)
        o, i_ref, _, _ = L.oracle_moe(x)
        assert np.array_equal(gi.cpu().numpy(), i_ref)
        assert synth.rel_l2(go.cpu().numpy(), o) < TOL
    layer.check()
    layer.close()


def test_prefill_graph_survives_growth(torch, k3x):
    """A prefill graph recorded over the layer's buffers stays valid after an eager call
    with more tokens grows them (the old buffers are kept, not freed), and a capture that
    would need to grow them is refused with K3X_E_SHAPE instead of allocating inside the
    capture."""
    say("case: prefill T=24 graph, eager T=100 grows the buffers, replay still exact")
    L = synth.tiny(seed=36)
    layer = bank_layer(k3x, L)
    layer.reserve(24)
    T, H, K = 24, L.H, L.K
    xd = torch.empty((T, H), dtype=torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        layer.forward(out.data_ptr(), xd.data_ptr(), T, k3x.K3X_F32, stream=s.cuda_stream)
    torch.cuda.synchronize()
    n0 = layer.nbytes()
    xb = L.x(100, bf16=False, stream_sub=30)
    ob, ib, _ = dev_forward(torch, k3x, layer, xb)       # grows the prefill buffers
    assert layer.nbytes() > n0
    o, i_ref, _, _ = L.oracle_moe(xb)
    assert np.array_equal(ib, i_ref) and synth.rel_l2(ob, o) < TOL
    for r in range(2):
        x = L.x(T, bf16=False, stream_sub=31 + r)
        xd.copy_(torch.from_numpy(x))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        o, _, _, _ = L.oracle_moe(x)
        say(f"  replay {r}")
        assert synth.rel_l2(out.cpu().numpy(), o) < TOL
    # capturing a call that needs more than is reserved is refused
    big = layer.nbytes()
    T2 = 4000
    x2 = torch.zeros((T2, H), dtype=torch.float32, device="cuda")
    o2 = torch.empty((T2, H), dtype=torch.float32, device="cuda")
    s2 = torch.cuda.Stream()
    torch.cuda.synchronize()
    with pytest.raises(k3x.K3XError) as ei:
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2, stream=s2):
            layer.forward(o2.data_ptr(), x2.data_ptr(), T2, k3x.K3X_F32, stream=s2.cuda_stream)
    assert ei.value.status == -2
    torch.cuda.synchronize()
    assert layer.nbytes() == big
    layer.check()
    layer.close()
