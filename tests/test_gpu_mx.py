"""GPU parity of the opt-in MXFP8-activation prefill mode (k3x_moe_layer_set_prefill_mode,
K3X_PREFILL_MXFP8): the routed products on the scaled matrix cores, MXFP4 weights as
stored, activations quantised to MXFP8.

The mode has no reference counterpart; its oracle is ko_moe_mx (the reference's
arithmetic with the documented activation quantisation, pinned in test_oracle_mx.py).
Bar: selected experts bit-exact (the router is the exact path's); outputs against
ko_moe_mx token by token (check_mx: the matrix core's accumulation and E4M3 rounding
boundaries separate the two by about 1e-4 per token).  Against the exact reference arithmetic the mode is a few percent
away (the E4M3 quantisation), which the tests also check, so that a path that silently
ran exact would fail.
"""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, say, synth_layer

pytestmark = pytest.mark.gpu


def check_mx(out, o, label):
    """Against the MXFP8 oracle, token by token.  Two effects separate them, both far
    below the quantisation itself (about 5e-2 from the exact path):
      - the scaled matrix core sums a 64-product step in a fixed-point accumulator
        narrower than the products' range (measured on gfx950: bit-exact when a block's
        products span a few binades, 1.3e-5 of sum|products| on average when the codes
        span E4M3's whole range), where the oracle sums in double;
      - a gate/up output that lies within that difference of an E4M3 rounding boundary
        quantises one step apart, which moves its token by about 1e-3.
    So: the median token within 2e-4, at most a quarter of the tokens beyond 2e-3, none
    beyond 2e-2."""
    r = np.linalg.norm((out - o).astype(np.float64), axis=1) / np.maximum(
        np.linalg.norm(o.astype(np.float64), axis=1), 1e-30)
    say(f"  {label}: per-token rel_l2 median {np.median(r):.2e} max {r.max():.2e}, "
        f"tokens beyond 2e-3: {int((r > 2e-3).sum())} of {r.size}")
    assert np.median(r) < 2e-4
    assert np.mean(r > 2e-3) <= 0.25
    assert r.max() < 2e-2


def mx_layer(k3x, L, synthetic=False):
    layer = synth_layer(k3x, L) if synthetic else bank_layer(k3x, L)
    layer.set_prefill_mode(k3x.K3X_PREFILL_MXFP8)
    return layer


@pytest.mark.parametrize("T,bf16", [(9, False), (40, False), (40, True), (150, True)])
def test_mx_tiny_vs_mx_oracle(torch, k3x, T, bf16):
    say(f"case: MXFP8 prefill, tiny layer, T={T}, {'bf16' if bf16 else 'fp32'} input")
    L = synth.tiny(seed=11)
    layer = mx_layer(k3x, L)
    x = L.x(T, bf16=bf16, stream_sub=2)
    out, idx, wt = dev_forward(torch, k3x, layer, x, bf16=bf16)
    o, oi, ow, drops = L.oracle_moe_mx(x)
    e, _, _, _ = L.oracle_moe(x)
    assert drops == 0 and np.array_equal(idx, oi)
    np.testing.assert_allclose(wt, ow, rtol=1e-6)
    dist = synth.rel_l2(out, e)
    say(f"  rel_l2 vs the exact oracle {dist:.3e}")
    check_mx(out, o, "vs the MXFP8 oracle")
    assert 1e-3 < dist < 1e-1
    layer.close()


def test_mx_exact_mode_switch(torch, k3x):
    """Back to K3X_PREFILL_EXACT, the same layer gives the exact path's results again."""
    say("case: MXFP8 then exact mode on one layer")
    L = synth.tiny(seed=12)
    layer = mx_layer(k3x, L)
    x = L.x(30, bf16=False, stream_sub=4)
    om, _, _ = dev_forward(torch, k3x, layer, x)
    layer.set_prefill_mode(k3x.K3X_PREFILL_EXACT)
    oe, _, _ = dev_forward(torch, k3x, layer, x)
    e, _, _, _ = L.oracle_moe(x)
    assert synth.rel_l2(oe, e) < 1e-3
    assert synth.rel_l2(om, e) > 1e-3
    layer.close()


def test_mx_latent_layer(torch, k3x):
    """A LatentMoE layer (latent 128, SiTU 4/25, latent norm, 2 shared experts): z is
    quantised at the latent width."""
    say("case: MXFP8 prefill, tiny LatentMoE layer, T=33")
    L = synth.tiny_latent(seed=0)
    layer = mx_layer(k3x, L)
    x = L.x(33, bf16=False, stream_sub=6)
    out, idx, _ = dev_forward(torch, k3x, layer, x)
    o, oi, _, _ = L.oracle_moe_mx(x)
    assert np.array_equal(idx, oi)
    check_mx(out, o, "vs the MXFP8 oracle")
    layer.close()


def test_mx_refuses_special_scale_bytes(torch, k3x):
    """A layer holding an E8M0 byte outside 1..252 keeps the exact path: the matrix cores
    read byte 255 as NaN, the reference as zero."""
    say("case: MXFP8 mode refused for a layer with scale byte 255")
    L = synth.tiny(seed=13)
    L.expert(3)["s2"][0, 0] = 255
    layer = bank_layer(k3x, L)
    with pytest.raises(k3x.K3XError) as ei:
        layer.set_prefill_mode(k3x.K3X_PREFILL_MXFP8)
    assert ei.value.status == -2                     # K3X_E_SHAPE
    with pytest.raises(k3x.K3XError) as ei:
        layer.set_prefill_mode(7)
    assert ei.value.status == -1                     # K3X_E_ARG
    x = L.x(20, bf16=False)
    out, _, _ = dev_forward(torch, k3x, layer, x)
    e, _, _, _ = L.oracle_moe(x)
    assert synth.rel_l2(out, e) < 1e-3
    layer.close()


def test_mx_full_2048_zipf(torch, k3x):
    """The full-size layer, 2048 bf16 tokens, Zipf-skewed bias: routing of every token
    equal to the exact mode's, 257 tokens spread over the chunk against the MXFP8
    oracle, and the chunk within a few percent of the exact mode."""
    say("case: MXFP8 prefill, full-size layer, 2048 bf16 tokens, Zipf bias")
    L = synth.full(seed=3, zipf_alpha=1.0)
    layer = synth_layer(k3x, L)
    T = 2048
    x = L.x(T, bf16=True, stream_sub=5)
    oe, ie, _ = dev_forward(torch, k3x, layer, x, bf16=True)
    layer.set_prefill_mode(k3x.K3X_PREFILL_MXFP8)
    om, im, _ = dev_forward(torch, k3x, layer, x, bf16=True)
    assert np.array_equal(im, ie)
    dist = synth.rel_l2(om, oe)
    say(f"  rel_l2(MXFP8 mode, exact mode) over 2048 tokens = {dist:.3e}")
    assert 1e-3 < dist < 1e-1
    # 257 tokens spread over the chunk against the MXFP8 oracle, token by token
    sample = np.r_[np.arange(3, T, 8), T - 1]
    L.hold(np.unique(im[sample]))
    o, oi, _, _ = L.oracle_moe_mx(x[sample])
    L.release()
    assert np.array_equal(im[sample], oi)
    check_mx(om[sample], o, f"{sample.size} spread tokens vs the MXFP8 oracle")
    layer.close()


def test_mx_graph_replays(torch, k3x):
    """The MXFP8 prefill captured in a graph and replayed equals the eager call."""
    say("case: MXFP8 prefill under graph capture, tiny layer, T=24, 3 replays")
    L = synth.tiny(seed=14)
    layer = mx_layer(k3x, L)
    T = 24
    layer.reserve(T)
    x = L.x(T, bf16=False, stream_sub=8)
    xt = torch.from_numpy(x).cuda()
    out = torch.empty((T, L.H), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        layer.forward(out.data_ptr(), xt.data_ptr(), T, k3x.K3X_F32, stream=s.cuda_stream)
    torch.cuda.synchronize()
    want = out.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        layer.forward(out.data_ptr(), xt.data_ptr(), T, k3x.K3X_F32, stream=s.cuda_stream)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want)
    layer.close()
