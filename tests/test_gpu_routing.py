"""GPU routing edge cases through the C ABI, decode and prefill, against the oracle (which
is bitwise the reference's k3_router, k3_ops.c:1624-1719): exact ties between experts
(the lower index first), NaN and -inf choices (never taken), +inf choices (taken first),
fewer selectable experts than slots (the rounds that find nothing give index 0 and
weight 0), and an expert count that is not a multiple of the wave width."""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, say, synth_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3


def check(torch, k3x, L, label):
    layer = bank_layer(k3x, L)
    x = L.x(20, bf16=False, stream_sub=11)
    o, idx, wt, _ = L.oracle_moe(x)
    for T in (1, 3, 20):           # decode, decode, prefill
        out, i2, w2 = dev_forward(torch, k3x, layer, x[:T])
        assert np.array_equal(i2, idx[:T]), (label, T, i2, idx[:T])
        np.testing.assert_allclose(w2, wt[:T], rtol=1e-6)
        err = synth.rel_l2(out, o[:T])
        say(f"  {label} T={T} rel_l2={err:.3e}")
        assert err < TOL
    layer.close()
    return idx


def test_exact_ties_lower_index_first(torch, k3x):
    say("case: E=200 K=8, experts 3, 10, 150 with identical router rows and bias (ties)")
    L = synth.Layer(H=256, E=200, K=8, I=128, seed=31)
    for e in (10, 150):
        L.gate[e] = L.gate[3]
    L.bias[[3, 10, 150]] = 5.0             # certainly among the top-k
    L.gate[77] = L.gate[160]
    L.bias[77] = L.bias[160]                # a tie anywhere in the ranking
    idx = check(torch, k3x, L, "ties")
    for t in range(idx.shape[0]):
        assert list(idx[t][:3]) == [3, 10, 150]


def test_nan_and_infinite_choices(torch, k3x):
    say("case: tiny layer, bias NaN / -inf on some experts, +inf on one")
    L = synth.tiny(seed=32)
    L.bias[[1, 4]] = np.nan
    L.bias[[2, 9]] = -np.inf
    L.bias[12] = np.inf
    idx = check(torch, k3x, L, "nan/inf")
    assert not np.isin(idx, [1, 2, 4, 9]).any()
    assert (idx[:, 0] == 12).all()


def test_fewer_selectable_than_slots(torch, k3x):
    say("case: tiny layer, only three selectable experts for four slots")
    L = synth.tiny(seed=33)
    L.bias[:] = np.nan
    L.bias[[5, 9, 14]] = 0.0
    idx = check(torch, k3x, L, "few")
    for t in range(idx.shape[0]):
        assert sorted(idx[t][:3]) == [5, 9, 14] and idx[t][3] == 0


@pytest.mark.parametrize("T", [1, 2])
def test_wait_bound_reports_and_recovers(torch, k3x, T):
    """Failure handling of the decode wait, forced from the host: the selection's routing
    words are withheld and the bound set to 2 us, so every routed workgroup gives up (and
    exits), for one token as for several; the check reports K3X_E_WAIT once, and the next
    call with the defaults is valid."""
    say(f"case: decode wait bound forced (words withheld, 2 us), then restored, T={T}")
    L = synth.tiny(seed=34)
    layer = bank_layer(k3x, L)
    x = L.x(T, bf16=False, stream_sub=12)
    o, idx, _, _ = L.oracle_moe(x)
    layer.set_route_wait(200, publish=False)
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = torch.empty_like(xt)
    layer.forward(out.data_ptr(), xt.data_ptr(), T, k3x.K3X_F32)
    torch.cuda.synchronize()
    with pytest.raises(k3x.K3XError) as ei:
        layer.check()
    assert "gave up waiting" in str(ei.value)
    layer.check()                           # reported once
    layer.set_route_wait(100000000, publish=True)
    out2, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    assert synth.rel_l2(out2, o) < TOL
    layer.close()


@pytest.mark.parametrize("T", [1, 3])
def test_wait_bound_host_call_returns_wait(torch, k3x, T):
    """The host-pointer drop-in (k3x_moe, behind the reference binding's k3_moe_gpu) must
    not return success on a call whose routed workgroups gave up waiting: with the flag
    withheld it raises K3X_E_WAIT, and the next call with the defaults is valid."""
    say(f"case: host-pointer k3x_moe with the decode wait forced, then restored, T={T}")
    L = synth.tiny(seed=35)
    layer = bank_layer(k3x, L)
    x = L.x(T, bf16=False, stream_sub=13)
    o, idx, _, _ = L.oracle_moe(x)
    layer.set_route_wait(200, publish=False)
    with pytest.raises(k3x.K3XError) as ei:
        layer.moe(x)
    assert ei.value.status == -7, str(ei.value)
    layer.check()                           # the host call cleared the word
    layer.set_route_wait(100000000, publish=True)
    out, il, _ = layer.moe(x)
    assert np.array_equal(il, idx[-1])
    assert synth.rel_l2(out, o) < TOL
    layer.close()


def test_prefill_router_sequential_chain_bitwise(torch, k3x):
    """The prefill router's logits are the reference's single double chain over
    i = 0 .. H-1 (k3_ops.c:1666-1688) bit for bit.  The router rows are equal at columns
    p and p+1 and every token carries +2^40 and -2^40 there, so the pair cancels but first
    rounds away low bits of the partial sum it meets, which depends on the summation order.
    With renorm off and scale 1 the routing weights are the sigmoid scores themselves and
    are compared bitwise with the oracle's.  E = 100 and T = 70 are not multiples of the
    router's 48-expert and 64-token blocks.  Teeth: on the same data a four-chain order
    changes the float logits of most pairs."""
    import oracle_lib as ol
    say("case: prefill router on cancelling data, E=100 H=1024 T=70, weights bitwise")
    H, E, K, T, p = 1024, 100, 8, 70, 512
    L = synth.Layer(H=H, E=E, K=K, I=128, seed=41, renorm=0, routed_scale=1.0)
    L.gate[:, p + 1] = L.gate[:, p]
    rng = np.random.default_rng(41)
    x = rng.standard_normal((T, H)).astype(np.float32)
    sgn = np.where(rng.integers(0, 2, T) == 1, 1.0, -1.0).astype(np.float32)
    x[:, p] = sgn * np.float32(2.0 ** 40)
    x[:, p + 1] = -sgn * np.float32(2.0 ** 40)
    # teeth (CPU): the sequential chain against a four-chain order
    W64, X64 = L.gate.astype(np.float64), x.astype(np.float64)
    seq = np.zeros((T, E))
    ch = np.zeros((4, T, E))
    for i in range(H):
        term = X64[:, i:i + 1] * W64[:, i][None, :]
        seq = seq + term
        ch[i % 4] = ch[i % 4] + term
    four = ((ch[0] + ch[1]) + ch[2]) + ch[3]
    differ = np.mean(seq.astype(np.float32) != four.astype(np.float32))
    say(f"  float logits that a four-chain order changes: {differ:.1%}")
    assert differ > 0.2
    layer = bank_layer(k3x, L)
    _, idx, wt = dev_forward(torch, k3x, layer, x)
    ri = np.empty((T, K), np.int32)
    rw = np.empty((T, K), np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_router(ol.ptr(ri[t], ol.I32P), ol.ptr(rw[t], ol.F32P),
                              ol.ptr(xt, ol.F32P), ol.ptr(L.gate, ol.F32P),
                              ol.ptr(L.bias, ol.F32P), H, E, K, 0, 1.0)
    assert np.array_equal(idx, ri)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    layer.close()


def cancelling_tokens(H, T, p, seed, big, bf16):
    """T tokens N(0, 1) (bf16 values when bf16) carrying +big and -big (a random sign a
    token) at columns p and p + 1."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    if bf16:
        x = synth.bf16_to_f32(synth.f32_to_bf16(x.ravel())).reshape(T, H)
    sgn = np.where(rng.integers(0, 2, T) == 1, 1.0, -1.0).astype(np.float32)
    x[:, p] = sgn * np.float32(big)
    x[:, p + 1] = -sgn * np.float32(big)
    return x


def four_chain_changes(W, x):
    """Fraction of float logits that summing in four interleaved chains instead of the
    reference's single chain changes (the test data's teeth)."""
    W64, X64 = W.astype(np.float64), x.astype(np.float64)
    seq = np.zeros((x.shape[0], W.shape[0]))
    ch = np.zeros((4,) + seq.shape)
    for i in range(x.shape[1]):
        term = X64[:, i:i + 1] * W64[:, i][None, :]
        seq = seq + term
        ch[i % 4] = ch[i % 4] + term
    four = ((ch[0] + ch[1]) + ch[2]) + ch[3]
    return np.mean(seq.astype(np.float32) != four.astype(np.float32))


def oracle_routes(L, x):
    import oracle_lib as ol
    T, H = x.shape
    ri = np.empty((T, L.K), np.int32)
    rw = np.empty((T, L.K), np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_router(ol.ptr(ri[t], ol.I32P), ol.ptr(rw[t], ol.F32P),
                              ol.ptr(xt, ol.F32P), ol.ptr(L.gate, ol.F32P),
                              ol.ptr(L.bias, ol.F32P), H, L.E, L.K, L.renorm, L.routed_scale)
    return ri, rw


@pytest.mark.parametrize("big", [2.0 ** 28, 2.0 ** 40])
@pytest.mark.parametrize("H,E,bf16", [(1024, 100, False), (1024, 100, True), (7168, 384, True)])
@pytest.mark.parametrize("T", [1, 8])
def test_decode_router_sequential_chain_bitwise(torch, k3x, T, H, E, bf16, big):
    """The decode path's routing is the reference's (k3_ops.c:1624-1719) bit for bit where
    its parallel logit sums round differently from the reference's single double chain:
    every logit whose float is not proven equal and that could change the selection or a
    selected weight is worked out again as that chain.  The router rows are equal at
    columns p and p + 1 and every token carries +big and -big there, so the pair cancels
    but first rounds away low bits of the partial sum it meets.  Renorm off and scale 1:
    the weights are the sigmoid scores, compared bitwise with the oracle's.  T = 1 runs
    k1_router_bset, T = 8 k1_router_mt; 2^28 changes about one float logit in eight
    (some experts proven, some worked out again), 2^40 nearly all."""
    say(f"case: decode router on cancelling data, H={H} E={E} T={T} bf16={bf16} big=2^"
        f"{int(np.log2(big))}, weights bitwise")
    K, p = 8, H // 2
    L = synth.Layer(H=H, E=E, K=K, I=128, seed=61, renorm=0, routed_scale=1.0)
    L.gate[:, p + 1] = L.gate[:, p]
    x = cancelling_tokens(H, T, p, 61 + T, big, bf16)
    if H == 1024:
        differ = four_chain_changes(L.gate, x)
        say(f"  float logits that a four-chain order changes: {differ:.1%}")
        assert differ > 0.05
    layer = bank_layer(k3x, L)
    _, idx, wt = dev_forward(torch, k3x, layer, x, bf16=bf16)
    n = layer.exact_count()
    ri, rw = oracle_routes(L, x)
    say(f"  logits worked out as the reference's chain: {n} of {T * E}")
    assert n > 0
    assert np.array_equal(idx, ri)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    layer.close()


@pytest.mark.parametrize("T", [1, 3])
def test_decode_router_sequential_chain_bitwise_norm(torch, k3x, T):
    """The same for the stacked layers' decode calls, whose router reads the RMSNorm of h
    worked out in its own launch: norm weights of 2^30 at the cancelling columns, so that
    the normalised pair still dominates every partial sum.  The routing is read back with
    k3x_moe_layer_last_route and compared bitwise with the oracle's RMSNorm then router."""
    import oracle_lib as ol
    say(f"case: stacked decode router on cancelling data, T={T}, weights bitwise")
    H, E, K, p, eps = 1024, 100, 8, 512, 1e-5
    L = synth.Layer(H=H, E=E, K=K, I=128, seed=71, renorm=0, routed_scale=1.0)
    L.gate[:, p + 1] = L.gate[:, p]
    nw = np.ones(H, np.float32)
    nw[p] = nw[p + 1] = np.float32(2.0 ** 30)
    x = cancelling_tokens(H, T, p, 71 + T, 2.0 ** 10, False)
    y = np.empty_like(x)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_rmsnorm(ol.ptr(y[t], ol.F32P), ol.ptr(xt, ol.F32P), ol.ptr(nw, ol.F32P),
                               H, eps)
    differ = four_chain_changes(L.gate, y)
    say(f"  float logits that a four-chain order changes: {differ:.1%}")
    assert differ > 0.05
    layer = bank_layer(k3x, L)
    nd = torch.from_numpy(nw).cuda()
    S = k3x.Stack([layer], [nd.data_ptr()], eps=eps, max_T=8)
    h = torch.from_numpy(x).cuda()
    S.forward(h.data_ptr(), T, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    idx, wt = layer.last_route(T)
    n = layer.exact_count()
    ri, rw = oracle_routes(L, y)
    say(f"  logits worked out as the reference's chain: {n} of {T * E}")
    assert n > 0
    assert np.array_equal(idx, ri)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    S.close()
    layer.close()


@pytest.mark.parametrize("T", [1, 3])
def test_stacked_router_on_norm_window_rows_bitwise(torch, k3x, T):
    """The stacked layers' decode router reads the RMSNorm of h worked out in its own
    launch; on rows at the scale's rounding midpoints (synth.rms_window_row) that launch
    sums the squares again as the reference's chain, so the normalised rows, and with
    them the routing weights (renorm off, scale 1), are the reference's bit for bit."""
    import oracle_lib as ol
    say(f"case: stacked decode router on RMSNorm window rows, T={T}, weights bitwise")
    H, E, K, eps = 1024, 100, 8, 1e-5
    L = synth.Layer(H=H, E=E, K=K, I=128, seed=81, renorm=0, routed_scale=1.0)
    nw = (1 + 0.1 * np.random.default_rng(81).standard_normal(H)).astype(np.float32)
    x = np.stack([synth.rms_window_row(H, eps, 200 + t) for t in range(T)])
    y = np.empty_like(x)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_rmsnorm(ol.ptr(y[t], ol.F32P), ol.ptr(xt, ol.F32P), ol.ptr(nw, ol.F32P),
                               H, eps)
    layer = bank_layer(k3x, L)
    nd = torch.from_numpy(nw).cuda()
    S = k3x.Stack([layer], [nd.data_ptr()], eps=eps, max_T=8)
    h = torch.from_numpy(x).cuda()
    S.forward(h.data_ptr(), T, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    idx, wt = layer.last_route(T)
    ri, rw = oracle_routes(L, y)
    assert np.array_equal(idx, ri)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    S.close()
    layer.close()


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("H,E", [(1024, 100), (7168, 384)])
def test_decode_router_same_bits_for_any_token_count(torch, k3x, bf16, H, E):
    """The decode router's logits do not depend on how many tokens a call carries: a call
    of T = 2 .. 8 tokens (the multi-token kernel, x staged in LDS, several experts a
    workgroup) gives each token the routing weights of its own T = 1 call (k1_router_bset)
    bit for bit, and the same experts.  Renorm off and scale 1, so the weights are the
    sigmoid scores themselves.  E = 100 is not a multiple of the experts per workgroup."""
    say(f"case: decode router, T=1 calls against T=2..8 calls, H={H} E={E} bf16={bf16}")
    L = synth.Layer(H=H, E=E, K=8, I=128, seed=51, renorm=0, routed_scale=1.0)
    layer = synth_layer(k3x, L)
    x = L.x(8, bf16=bf16, stream_sub=12)
    ones = [dev_forward(torch, k3x, layer, x[t:t + 1], bf16=bf16) for t in range(8)]
    i1 = np.concatenate([o[1] for o in ones])
    w1 = np.concatenate([o[2] for o in ones])
    for T in (2, 3, 5, 8):
        _, iT, wT = dev_forward(torch, k3x, layer, x[:T], bf16=bf16)
        assert np.array_equal(iT, i1[:T]), T
        assert np.array_equal(wT.view(np.uint32), w1[:T].view(np.uint32)), T
    layer.close()


def dev_route(torch, k3x, layer, x, bf16=False):
    """k3x_moe_route on device copies; (idx, wt) on the host."""
    T = x.shape[0]
    K = layer.cfg.topk
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    if bf16:
        xt = xt.to(torch.bfloat16)
    idx = torch.full((T, K), -7, dtype=torch.int32, device="cuda")
    wt = torch.full((T, K), -7.0, dtype=torch.float32, device="cuda")
    layer.route(idx.data_ptr(), wt.data_ptr(), xt.data_ptr(), T,
                k3x.K3X_BF16 if bf16 else k3x.K3X_F32, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), wt.cpu().numpy()


@pytest.mark.parametrize("bf16", [False, True])
def test_route_alone_matches_oracle_and_forward(torch, k3x, bf16):
    """k3x_moe_route (the router alone, k3_router k3_ops.c:1624-1719) gives the oracle's
    experts and weights bit for bit at 1, 3 and 20 tokens, with NaN, -inf and +inf biases
    and a tie in the ranking, and the same routing k3x_moe_forward reports for the same
    tokens."""
    say(f"case: router alone, E=200 K=8, ties and NaN/inf biases, bf16={bf16}")
    L = synth.Layer(H=256, E=200, K=8, I=128, seed=71)
    L.gate[77] = L.gate[160]
    L.bias[77] = L.bias[160]
    L.bias[[5, 9]] = np.nan
    L.bias[[11]] = -np.inf
    L.bias[42] = np.inf
    x = L.x(20, bf16=bf16, stream_sub=71)
    layer = bank_layer(k3x, L)
    ri, rw = oracle_routes(L, x)
    for T in (1, 3, 20):
        idx, wt = dev_route(torch, k3x, layer, x[:T], bf16=bf16)
        assert np.array_equal(idx, ri[:T]), (T, idx, ri[:T])
        assert np.array_equal(wt.view(np.uint32), rw[:T].view(np.uint32))
        _, i2, w2 = dev_forward(torch, k3x, layer, x[:T], bf16=bf16)
        assert np.array_equal(i2, idx) and np.array_equal(w2.view(np.uint32), wt.view(np.uint32))
        say(f"  T={T}: bitwise")
    assert (ri[:, 0] == 42).all()
    layer.close()


def test_route_alone_cancelling_data_bitwise(torch, k3x):
    """The router alone on the cancelling data of the prefill router test (a four-chain
    order changes most float logits): weights bitwise the oracle's, renorm off."""
    say("case: router alone on cancelling data, E=100 H=1024 T=70, weights bitwise")
    H, E, K, T, p = 1024, 100, 8, 70, 512
    L = synth.Layer(H=H, E=E, K=K, I=128, seed=72, renorm=0, routed_scale=1.0)
    L.gate[:, p + 1] = L.gate[:, p]
    x = cancelling_tokens(H, T, p, 72, 2.0 ** 40, False)
    layer = bank_layer(k3x, L)
    idx, wt = dev_route(torch, k3x, layer, x)
    ri, rw = oracle_routes(L, x)
    assert np.array_equal(idx, ri)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    layer.close()


def test_route_alone_full_shape(torch, k3x):
    """The router alone at the K2 shape (7168 x 384, top-8, Zipf-skewed biases), 300 bf16
    tokens: experts and weights bitwise the oracle's."""
    say("case: router alone, full K2 router, 300 bf16 tokens, Zipf-skewed")
    L = synth.full(seed=73, zipf_alpha=1.0)
    layer = synth_layer(k3x, L)
    x = L.x(300, bf16=True, stream_sub=73)
    idx, wt = dev_route(torch, k3x, layer, x, bf16=True)
    ri, rw = oracle_routes(L, x)
    assert np.array_equal(idx, ri)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    layer.close()
