"""GPU parity of the K3 LatentMoE form against the oracle, through the C ABI.

Same bar as the K2-class layer: every selected expert index bit-exact, outputs within
TOL relative L2 of the oracle (itself pinned bit for bit to the compiled reference's
k3_moe on these layers, and to the reference's moe.json fixture).  The latent form adds
the down projection to the latent width, experts there with SiTU-GLU (betas 4 and 25),
the RMSNorm of the routed aggregate, the up projection and two full-width shared experts.
"""
import os

import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, host_layer, per_token_rel, say, synth_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3          # relative L2
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def tiny_lat(torch, k3x):
    L = synth.tiny_latent(seed=0)
    layer = bank_layer(k3x, L)
    yield L, layer
    layer.close()


def test_latent_golden_vectors(torch, k3x, tiny_lat):
    say("case: tiny latent layer vs compiled-reference golden vectors (k3_tiny.npz)")
    L, layer = tiny_lat
    g = np.load(os.path.join(GOLD, "k3_tiny.npz"))
    x = L.x(int(g["T"]), bf16=False)
    for T in (1, 2, 6):
        out, idx, wt = dev_forward(torch, k3x, layer, x[:T])
        assert np.array_equal(idx, g["idx"][:T])
        np.testing.assert_allclose(wt, g["wt"][:T], rtol=1e-6)
        err = synth.rel_l2(out, g["out"][:T])
        say(f"  T={T} rel_l2={err:.3e}")
        assert err < TOL


@pytest.mark.parametrize("T,bf16", [(1, False), (3, True), (8, False)])
def test_latent_tiny_vs_oracle(torch, k3x, tiny_lat, T, bf16):
    say(f"case: tiny latent layer T={T} bf16={bf16} vs oracle")
    L, layer = tiny_lat
    x = L.x(T, bf16=bf16, stream_sub=10 + T)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=bf16)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL


def test_latent_resid_and_grouped_call(torch, k3x, tiny_lat):
    """resid + MoE, and T = 20 (more tokens than one decode call takes)."""
    say("case: tiny latent layer, T=20 with residual")
    L, layer = tiny_lat
    x = L.x(20, bf16=False, stream_sub=30)
    r = L.x(20, bf16=False, stream_sub=31)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x, resid=r)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o + r)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL


@pytest.mark.parametrize("norm,shared", [(0, 2), (1, 0)])
def test_latent_variants(torch, k3x, norm, shared):
    """Without the latent norm; without shared experts (the up projection alone)."""
    say(f"case: tiny latent layer, latent_norm={norm}, n_shared={shared}")
    L = synth.tiny_latent(seed=6, latent_norm=norm, n_shared=shared)
    layer = bank_layer(k3x, L)
    x = L.x(4, bf16=False)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    layer.close()


@pytest.mark.parametrize("H,LT,I,NS", [(2048, 2048, 128, 2), (512, 512, 1024, 2)])
def test_latent_set_placements(torch, k3x, H, LT, I, NS):
    """T = 8 on shapes whose up-projection sets take the other placements: the aggregates'
    set too large for the LDS with the shared set staged (2048/2048/128), and the
    aggregates' set worked out in the workgroup with the shared set read from memory
    (512/512/1024)."""
    say(f"case: latent layer H={H} latent={LT} I={I} shared={NS}, T=8")
    L = synth.Layer(H=H, E=16, K=4, I=I, n_shared=NS, latent=LT, latent_norm=1,
                    situ_b1=4.0, situ_b2=25.0, routed_scale=1.0, seed=11)
    layer = bank_layer(k3x, L)
    x = L.x(8, bf16=False)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    layer.close()


def test_latent_host_dropin(torch, k3x):
    say("case: tiny latent layer, host-pointer k3x_moe vs oracle")
    L = synth.tiny_latent(seed=7)
    layer = bank_layer(k3x, L)
    x = L.x(5, bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    out, il, wl = layer.moe(x, prefill=False)
    assert np.array_equal(il, idx[-1])
    assert synth.rel_l2(out, o) < TOL
    layer.close()


def test_latent_synthetic_equals_host_generator(torch, k3x):
    say("case: device-generated synthetic latent layer equals the host generator")
    L = synth.tiny_latent(seed=8)
    layer = synth_layer(k3x, L)
    for e in (0, 9):
        d = layer.read_expert(e)
        for k, v in L.expert(e).items():
            assert np.array_equal(d[k], v), (e, k)
    x = L.x(2, bf16=False)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    assert synth.rel_l2(out, o) < TOL
    layer.close()


# ------------------------------------------------------------------ the K3 shape
@pytest.fixture(scope="module")
def k3_layer(torch, k3x):
    say("building the K3-shape synthetic latent layer (896 experts) on the device")
    L = synth.k3(seed=1)
    layer = synth_layer(k3x, L)
    yield L, layer
    layer.close()


def test_k3_decode_b1(torch, k3x, k3_layer):
    say("case: K3 shape (H 7168, latent 3584, top-16 of 896), decode b=1, 2 tokens")
    L, layer = k3_layer
    x = L.x(2, bf16=True, stream_sub=2)
    o, idx, wt, _ = L.oracle_moe(x)
    for t in range(2):
        out, i2, w2 = dev_forward(torch, k3x, layer, x[t:t + 1], bf16=True)
        assert np.array_equal(i2[0], idx[t])
        np.testing.assert_allclose(w2[0], wt[t], rtol=1e-6)
        err = synth.rel_l2(out, o[t:t + 1])
        say(f"  token {t}: rel_l2={err:.3e}")
        assert err < TOL


def test_k3_decode_b2(torch, k3x, k3_layer):
    say("case: K3 shape, T=2 in one call vs oracle")
    L, layer = k3_layer
    x = L.x(2, bf16=False, stream_sub=5)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL


@pytest.mark.parametrize("T", [3, 4, 6])
def test_k3_decode_multi(torch, k3x, k3_layer, T):
    """T = 3..5 take the down products over parts without the activation sets in LDS,
    T = 6..7 take k3_down2 with parts; both feed k4_latent_norm (the aggregates past the
    LDS) at this shape."""
    say(f"case: K3 shape, T={T} in one call vs oracle")
    L, layer = k3_layer
    x = L.x(T, bf16=True, stream_sub=80 + T)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=True)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  unique experts {len(np.unique(idx))}, rel_l2={err:.3e}")
    assert err < TOL


def test_k3_decode_b8(torch, k3x, k3_layer):
    say("case: K3 shape, T=8 in one call vs oracle")
    L, layer = k3_layer
    x = L.x(8, bf16=True, stream_sub=3)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=True)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  unique experts {len(np.unique(idx))}, rel_l2={err:.3e}")
    assert err < TOL


# ------------------------------------------------------------------ prefill (T > 8)
def decode_forward(torch, k3x, layer, x, bf16):
    """The same tokens through the decode path, 8 at a time."""
    outs, idxs = [], []
    for t0 in range(0, x.shape[0], 8):
        o, i, _ = dev_forward(torch, k3x, layer, x[t0:t0 + 8], bf16=bf16)
        outs.append(o); idxs.append(i)
    return np.concatenate(outs), np.concatenate(idxs)


@pytest.mark.parametrize("T,bf16", [(9, False), (37, True), (130, False)])
def test_latent_prefill_vs_oracle(torch, k3x, tiny_lat, T, bf16):
    say(f"case: tiny latent layer prefill T={T} bf16={bf16} vs oracle")
    L, layer = tiny_lat
    x = L.x(T, bf16=bf16, stream_sub=50 + T)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=bf16)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL


@pytest.mark.parametrize("norm,shared", [(0, 2), (1, 0)])
def test_latent_prefill_variants(torch, k3x, norm, shared):
    say(f"case: tiny latent layer prefill T=40, latent_norm={norm}, n_shared={shared}, resid")
    L = synth.tiny_latent(seed=13, latent_norm=norm, n_shared=shared)
    layer = bank_layer(k3x, L)
    x = L.x(40, bf16=False)
    r = L.x(40, bf16=False, stream_sub=70)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x, resid=r)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o + r)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    layer.close()


def test_k3_prefill_256(torch, k3x, k3_layer):
    """The K3 shape, one call of 256 bf16 tokens: routing of every token against the
    oracle's router, every token against the decode path and against the whole layer on
    the host (the reference's k3_moe_prefill), each within TOL."""
    import oracle_lib as ol
    say("case: K3 shape prefill, 256 bf16 tokens")
    L, layer = k3_layer
    T = 256
    x = L.x(T, bf16=True, stream_sub=6)
    out, idx, wt = dev_forward(torch, k3x, layer, x, bf16=True)
    ri = np.empty((T, L.K), np.int32)
    rw = np.empty((T, L.K), np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_router(ol.ptr(ri[t], ol.I32P), ol.ptr(rw[t], ol.F32P),
                              ol.ptr(xt, ol.F32P), ol.ptr(L.gate, ol.F32P),
                              ol.ptr(L.bias, ol.F32P), L.H, L.E, L.K, 1, 1.0)
    assert np.array_equal(idx, ri)
    np.testing.assert_allclose(wt, rw, rtol=1e-6)
    say(f"  routing of all {T} tokens equals the oracle's; experts used "
        f"{len(np.unique(idx))}")
    o2, i2 = decode_forward(torch, k3x, layer, x, True)
    assert np.array_equal(idx, i2)
    err = synth.rel_l2(out, o2)
    say(f"  rel_l2(prefill, decode) over {T} tokens = {err:.3e}")
    assert err < 1e-5
    # every token against the whole layer on the host, token by token
    o, what = host_layer(L, x, ri)
    r = per_token_rel(out, o)
    say(f"  {T} tokens against {what}: per-token rel_l2 median {np.median(r):.2e} "
        f"max {r.max():.2e}")
    assert r.max() < TOL
