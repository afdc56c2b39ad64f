"""Stacked layers through the C ABI: h = h + MoE_l(RMSNorm_l(h)) per layer, replayed from
a HIP graph, against the oracle applying the same steps on the host (ko_rmsnorm, then
the oracle MoE of each layer, then the residual add)."""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, say, synth_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3
EPS = 1e-5


def oracle_stack(layers, norms, h):
    from oracle_lib import F32P, oracle, ptr
    h = np.array(h, np.float32)
    for L, w in zip(layers, norms):
        y = np.empty_like(h)
        for t in range(h.shape[0]):
            ht = np.ascontiguousarray(h[t])
            oracle().ko_rmsnorm(ptr(y[t], F32P), ptr(ht, F32P), ptr(w, F32P), h.shape[1], EPS)
        o, _, _, _ = L.oracle_moe(y)
        h = (h + o).astype(np.float32)
    return h


@pytest.fixture(scope="module")
def tiny_stack(torch, k3x):
    Ls = [synth.tiny(seed=20 + l) for l in range(3)]
    rng = np.random.default_rng(5)
    norms = [(1 + 0.1 * rng.standard_normal(Ls[0].H)).astype(np.float32) for _ in Ls]
    layers = [bank_layer(k3x, L) for L in Ls]
    nd = [torch.from_numpy(w).cuda() for w in norms]
    yield Ls, norms, layers, nd
    for l in layers:
        l.close()


@pytest.mark.parametrize("T", [1, 5, 12])
def test_stack_vs_oracle(torch, k3x, tiny_stack, T):
    say(f"case: 3 tiny layers stacked, T={T}, graph replay vs oracle")
    Ls, norms, layers, nd = tiny_stack
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=16)
    h0 = Ls[0].x(T, bf16=False, stream_sub=40 + T) * 2.0
    h = torch.from_numpy(h0).cuda()
    S.forward(h.data_ptr(), T, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = oracle_stack(Ls, norms, h0)
    err = synth.rel_l2(h.cpu().numpy(), want)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    S.close()


def test_stack_graph_replays(torch, k3x, tiny_stack):
    """One recorded graph replayed on new inputs, with eager work between replays; every
    replay checked."""
    say("case: stacked graph replayed 4 times with eager copies between")
    Ls, norms, layers, nd = tiny_stack
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=4)
    T = 2
    h = torch.empty((T, Ls[0].H), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    for r in range(4):
        x = Ls[0].x(T, bf16=False, stream_sub=60 + r)
        h.copy_(torch.from_numpy(x).cuda())
        S.forward(h.data_ptr(), T, s.cuda_stream)
        torch.cuda.synchronize()
        err = synth.rel_l2(h.cpu().numpy(), oracle_stack(Ls, norms, x))
        say(f"  replay {r}: rel_l2={err:.3e}")
        assert err < TOL
    S.close()


@pytest.mark.parametrize("T", [1, 3])
def test_stack_fused_norm_equals_separate_norm(torch, k3x, tiny_stack, T):
    """Decode-sized calls work the RMSNorm out inside the router launch; the result must be
    bitwise what a separate k3x_rmsnorm followed by the MoE call gives."""
    say(f"case: 3 tiny layers, T={T}, fused norm vs k3x_rmsnorm + forward, bitwise")
    Ls, norms, layers, nd = tiny_stack
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=8)
    h0 = Ls[0].x(T, bf16=False, stream_sub=90 + T) * 3.0
    h = torch.from_numpy(h0).cuda()
    s = torch.cuda.current_stream().cuda_stream
    S.forward(h.data_ptr(), T, s)
    ref = torch.from_numpy(h0).cuda()
    y = torch.empty_like(ref)
    for L, w in zip(layers, nd):
        k3x.rmsnorm(y.data_ptr(), ref.data_ptr(), w.data_ptr(), Ls[0].H, T, EPS, s)
        L.forward(ref.data_ptr(), y.data_ptr(), T, k3x.K3X_F32, ref.data_ptr(), 0, 0, s)
    torch.cuda.synchronize()
    assert torch.equal(h, ref)
    S.close()


def test_stack_rejects_too_many_tokens(torch, k3x, tiny_stack):
    Ls, norms, layers, nd = tiny_stack
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=2)
    h = torch.zeros((3, Ls[0].H), dtype=torch.float32, device="cuda")
    with pytest.raises(k3x.K3XError):
        S.forward(h.data_ptr(), 3, torch.cuda.current_stream().cuda_stream)
    S.close()


# ------------------------------------------------------------------ the full width
@pytest.fixture(scope="module")
def full_stack(torch, k3x):
    """Three full-size K2-class layers (H 7168, 384 experts top-8, I 2048; seeds 10 + l),
    generated on the device, with RMSNorm weights 1 + N(0, 0.1)."""
    say("building 3 full-size synthetic layers (27 GB) on the device")
    Ls = [synth.full(seed=10 + l, layer=l) for l in range(3)]
    rng = np.random.default_rng(6)
    norms = [(1 + 0.1 * rng.standard_normal(Ls[0].H)).astype(np.float32) for _ in Ls]
    layers = [synth_layer(k3x, L) for L in Ls]
    nd = [torch.from_numpy(w).cuda() for w in norms]
    yield Ls, norms, layers, nd
    for l in layers:
        l.close()


@pytest.mark.parametrize("T", [1, 3])
def test_full_stack_graph_vs_oracle(torch, k3x, full_stack, T):
    """The stacked-layer sequence at the benchmark's full width (H 7168): the first call
    records the graph, the next two replay it on new tokens; every call against the oracle
    applying ko_rmsnorm, the oracle MoE of each layer and the residual add on the host
    (k3_decoder_layer_core's MoE half, k3_ops.c:2559-2589)."""
    Ls, norms, layers, nd = full_stack
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=8)
    h = torch.empty((T, Ls[0].H), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    for r in range(3):
        say(f"case: 3 full-size layers stacked, T={T}, call {r} ({'record' if r == 0 else 'replay'})")
        h0 = Ls[0].x(T, bf16=False, stream_sub=110 + 10 * T + r) * 2.0
        h.copy_(torch.from_numpy(h0).cuda())
        S.forward(h.data_ptr(), T, s.cuda_stream)
        torch.cuda.synchronize()
        for l in layers:
            l.check()
        want = oracle_stack(Ls, norms, h0)
        err = synth.rel_l2(h.cpu().numpy(), want)
        say(f"  rel_l2={err:.3e}")
        assert err < TOL
    S.close()


@pytest.mark.parametrize("T", [1, 3])
def test_full_stack_fused_norm_bitwise(torch, k3x, full_stack, T):
    """At H 7168 the RMSNorm worked out inside the router launch gives bitwise what a
    separate k3x_rmsnorm followed by the MoE call gives, layer after layer."""
    say(f"case: 3 full-size layers, T={T}, fused norm vs k3x_rmsnorm + forward, bitwise")
    Ls, norms, layers, nd = full_stack
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=8)
    h0 = Ls[0].x(T, bf16=False, stream_sub=150 + T) * 3.0
    h = torch.from_numpy(h0).cuda()
    s = torch.cuda.current_stream().cuda_stream
    S.forward(h.data_ptr(), T, s)
    ref = torch.from_numpy(h0).cuda()
    y = torch.empty_like(ref)
    for L, w in zip(layers, nd):
        k3x.rmsnorm(y.data_ptr(), ref.data_ptr(), w.data_ptr(), Ls[0].H, T, EPS, s)
        L.forward(ref.data_ptr(), y.data_ptr(), T, k3x.K3X_F32, ref.data_ptr(), 0, 0, s)
    torch.cuda.synchronize()
    assert torch.equal(h, ref)
    S.close()


def test_full_stack_8_layers_per_layer(torch, k3x):
    """Eight full-size layers (the stack the benchmark replays: seeds 10 + l, RMSNorm
    weights 1 + N(0, 0.1) from the generator), one token (the benchmark's first): the
    replayed stack equals per-layer calls (k3x_rmsnorm, then the MoE call with the
    residual, its selection returned) bit for bit, and at every layer, on that layer's
    own input, the RMSNorm is the oracle's bit for bit, the selected experts are the
    oracle router's (weights to float rounding), and the layer's MoE output is within TOL
    of the oracle's whole layer."""
    import oracle_lib as ol
    NL, H = 8, 7168
    say(f"building {NL} full-size synthetic layers (75 GB) on the device")
    Ls = [synth.full(seed=10 + l, layer=l) for l in range(NL)]
    norms = [synth.normal_f32(H, synth.key(10 + l, l, synth.S_NORM), 1.0, 0.1)
             for l in range(NL)]
    layers = [synth_layer(k3x, L) for L in Ls]
    nd = [torch.from_numpy(w).cuda() for w in norms]
    s = torch.cuda.current_stream().cuda_stream
    S = k3x.Stack(layers, [w.data_ptr() for w in nd], eps=EPS, max_T=1)
    h0 = Ls[0].x(1, bf16=False, stream_sub=7)
    h = torch.from_numpy(h0).cuda()
    for r in range(2):                          # record, then replay on the same token
        h.copy_(torch.from_numpy(h0).cuda())
        S.forward(h.data_ptr(), 1, s)
    torch.cuda.synchronize()
    cur = torch.from_numpy(h0).cuda()
    y = torch.empty_like(cur)
    idx = torch.empty((1, Ls[0].K), dtype=torch.int32, device="cuda")
    wt = torch.empty((1, Ls[0].K), dtype=torch.float32, device="cuda")
    for l, (L, layer, w) in enumerate(zip(Ls, layers, nd)):
        inp = cur.cpu().numpy()
        k3x.rmsnorm(y.data_ptr(), cur.data_ptr(), w.data_ptr(), H, 1, EPS, s)
        layer.forward(cur.data_ptr(), y.data_ptr(), 1, k3x.K3X_F32, cur.data_ptr(),
                      idx.data_ptr(), wt.data_ptr(), s)
        torch.cuda.synchronize()
        layer.check()
        hin = np.empty_like(inp)
        ol.oracle().ko_rmsnorm(ol.ptr(hin[0], ol.F32P), ol.ptr(inp[0], ol.F32P),
                               ol.ptr(norms[l], ol.F32P), H, EPS)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), hin.view(np.uint32))
        o, oi, ow, _ = L.oracle_moe(hin)
        di = idx.cpu().numpy()
        assert np.array_equal(di, oi), (l, di, oi)
        np.testing.assert_allclose(wt.cpu().numpy(), ow, rtol=1e-6)
        moe = cur.cpu().numpy() - inp
        err = synth.rel_l2(moe, o)
        say(f"  layer {l}: experts {di[0].tolist()}, MoE rel_l2 {err:.2e}")
        assert err < TOL
    assert torch.equal(h, cur)
    S.close()
    for l in layers:
        l.close()
