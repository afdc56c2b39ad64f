"""GPU parity of the MoE block against the oracle, through the C ABI.

Parity bar: every selected expert index bit-exact (ties to the lower index), and
outputs within TOL relative L2 of the oracle's fp32/double arithmetic on the same seeded
inputs.  Full-size layers are built on the device by k3x_synth_layer_create and
regenerated element by element on the host for the oracle.
"""
import os

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3          # relative L2, the parity bar
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


from gpu_util import bank_layer, dev_forward, say, synth_layer  # noqa: E402


# ------------------------------------------------------------------ tiny layer
def test_tiny_golden_vectors(torch, k3x):
    say("case: tiny layer vs compiled-reference golden vectors (k2_tiny.npz)")
    g = np.load(os.path.join(GOLD, "k2_tiny.npz"))
    L = synth.tiny(seed=int(g["seed"]))
    layer = bank_layer(k3x, L)
    x = L.x(int(g["T"]), bf16=False)
    for T in (1, 2, 5, 8):
        out, idx, wt = dev_forward(torch, k3x, layer, x[:T])
        assert np.array_equal(idx, g["idx"][:T])
        np.testing.assert_allclose(wt, g["wt"][:T], rtol=1e-6)
        err = synth.rel_l2(out, g["out"][:T])
        say(f"  T={T} rel_l2={err:.3e}")
        assert err < TOL
    layer.close()


def test_tiny_host_dropin_matches_oracle(torch, k3x):
    say("case: tiny layer, host-pointer k3x_moe / k3x_moe_prefill vs oracle")
    L = synth.tiny(seed=3)
    layer = bank_layer(k3x, L)
    x = L.x(20, bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    for T in (1, 8, 20):
        for prefill in (False, True):
            out, il, wl = layer.moe(x[:T], prefill=prefill)
            if prefill and T > 1:
                # the batched k3_moe_prefill leaves idx/wt untouched (k3_ops.c:2018-2053)
                assert np.all(il == 0) and np.all(wl == 0)
            else:
                assert np.array_equal(il, idx[T - 1])
                np.testing.assert_allclose(wl, wt[T - 1], rtol=1e-6)
            assert synth.rel_l2(out, o[:T]) < TOL
    layer.close()


def test_tiny_tiling_round_trip(torch, k3x):
    say("case: tiled upload read back equals the uploaded bytes")
    L = synth.tiny(seed=5)
    layer = bank_layer(k3x, L)
    for e in (0, 7, 15):
        d = layer.read_expert(e)
        for k, v in L.expert(e).items():
            assert np.array_equal(d[k], v), (e, k)
    layer.close()


def test_tiny_synthetic_equals_host_generator(torch, k3x):
    say("case: device-generated synthetic layer equals the host generator")
    L = synth.tiny(seed=9)
    layer = synth_layer(k3x, L)
    for e in (0, 3, 15):
        d = layer.read_expert(e)
        for k, v in L.expert(e).items():
            assert np.array_equal(d[k], v), (e, k)
    x = L.x(4, bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    assert synth.rel_l2(out, o) < TOL
    layer.close()


def test_special_scale_bytes(torch, k3x):
    """E8M0 byte 255 zeroes its group (reference: k3_ops.c:3125-3132) and bytes far from
    the configs' 121..125 range still decode exactly."""
    say("case: tiny layer with scale bytes 255 and a wide exponent range")
    L = synth.tiny(seed=2, scale_lo=100, scale_hi=140)
    for e in range(L.E):
        d = L.expert(e)
        d["s1"][0, 1] = 255
        d["s3"][5, 0] = 255
        d["s2"][7, 2] = 255
    layer = bank_layer(k3x, L)
    x = L.x(3, bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL
    layer.close()


def test_resid_and_bf16_input(torch, k3x):
    say("case: resid + MoE and bf16 activations")
    L = synth.tiny(seed=4)
    layer = bank_layer(k3x, L)
    x = L.x(6, bf16=True)
    r = L.x(6, bf16=False, stream_sub=9)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x, bf16=True, resid=r)
    assert np.array_equal(i2, idx)
    assert synth.rel_l2(out, o + r) < TOL
    layer.close()


def test_rmsnorm_device(torch, k3x):
    say("case: RMSNorm on the device vs oracle")
    from oracle_lib import F32P, oracle, ptr
    rng = np.random.default_rng(0)
    T, n = 5, 7168
    x = rng.standard_normal((T, n)).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    want = np.empty_like(x)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        oracle().ko_rmsnorm(ptr(want[t], F32P), ptr(xt, F32P), ptr(w, F32P), n, 1e-5)
    xd = torch.from_numpy(x).cuda()
    wd = torch.from_numpy(w).cuda()
    yd = torch.empty_like(xd)
    k3x.rmsnorm(yd.data_ptr(), xd.data_ptr(), wd.data_ptr(), n, T, 1e-5,
                torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_allclose(yd.cpu().numpy(), want, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("n", [1024, 7168])
def test_rmsnorm_window_rows_bitwise(torch, k3x, n):
    """Rows whose sum of squares lies on the preimage of a float rounding midpoint of the
    scale (synth.rms_window_row): the kernel's tree sum cannot prove its float scale, sums
    the squares again as the reference's chain (k3_ops.c:135-136), and the normalised rows
    are the reference's bit for bit.  Two ordinary rows ride along."""
    say(f"case: RMSNorm on rows at the scale's rounding midpoints, n={n}, bitwise")
    from oracle_lib import F32P, oracle, ptr
    eps = 1e-5
    rng = np.random.default_rng(n)
    x = np.stack([synth.rms_window_row(n, eps, 100 + r) for r in range(4)] +
                 [rng.standard_normal(n).astype(np.float32) for _ in range(2)])
    T = x.shape[0]
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    want = np.empty_like(x)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        oracle().ko_rmsnorm(ptr(want[t], F32P), ptr(xt, F32P), ptr(w, F32P), n, eps)
    xd = torch.from_numpy(x).cuda()
    wd = torch.from_numpy(w).cuda()
    yd = torch.empty_like(xd)
    k3x.rmsnorm(yd.data_ptr(), xd.data_ptr(), wd.data_ptr(), n, T, eps,
                torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(yd.cpu().numpy().view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ full-size layer
@pytest.fixture(scope="module")
def full_normal(torch, k3x):
    say("building full-size synthetic layer (seed 1, normal bias) on the device")
    L = synth.full(seed=1)
    layer = synth_layer(k3x, L)
    yield L, layer
    layer.close()


def test_full_golden_vectors(torch, k3x, full_normal):
    """Against the compiled reference's own outputs at the K2 shape (k2_full.npz)."""
    say("case: full-size layer vs compiled-reference golden vectors")
    L, layer = full_normal
    g = np.load(os.path.join(GOLD, "k2_full.npz"))
    x = L.x(2, bf16=True, stream_sub=0)
    out, idx, wt = dev_forward(torch, k3x, layer, x, bf16=True)
    assert np.array_equal(idx, g["normal_idx"])
    np.testing.assert_allclose(wt, g["normal_wt"], rtol=1e-6)
    err = synth.rel_l2(out[:, ::16], g["normal_out16"])
    say(f"  rel_l2(sampled)={err:.3e}")
    assert err < TOL


def test_full_decode_b1_parity(torch, k3x, full_normal):
    say("case: full-size decode b=1, 6 tokens, vs oracle")
    L, layer = full_normal
    x = L.x(6, bf16=True, stream_sub=4)
    o, idx, wt, _ = L.oracle_moe(x)
    for t in range(6):
        out, i2, w2 = dev_forward(torch, k3x, layer, x[t:t + 1], bf16=True)
        assert np.array_equal(i2[0], idx[t])
        np.testing.assert_allclose(w2[0], wt[t], rtol=1e-6)
        err = synth.rel_l2(out, o[t:t + 1])
        say(f"  token {t}: rel_l2={err:.3e}")
        assert err < TOL


def test_full_verify_b8_zipf(torch, k3x):
    say("case: full-size T=8 verify batch, Zipf bias (alpha 1.0, s 1.1)")
    L = synth.full(seed=2, zipf_alpha=1.0)
    layer = synth_layer(k3x, L)
    x = L.x(8, bf16=True, stream_sub=1)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=True)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  unique experts {len(np.unique(idx))}, rel_l2={err:.3e}")
    assert 8 < len(np.unique(idx)) < 64
    assert err < TOL
    layer.close()


@pytest.mark.parametrize("T,bf16", [(3, False), (5, True)])
def test_full_decode_multi_token(torch, k3x, full_normal, T, bf16):
    """T = 3 and 5 at the full shape: the several-token kernels (each super-quad's B
    fragments staged once for the gate/up waves; the down products in 256-row workgroups
    over parts of the items, the parts added by k3_reduce) with B sets of 6 and 10
    columns, which fill the staging chunks only in part."""
    say(f"case: full-size decode T={T} ({'bf16' if bf16 else 'fp32'} tokens) vs oracle")
    L, layer = full_normal
    x = L.x(T, bf16=bf16, stream_sub=6 + T)
    o, idx, wt, _ = L.oracle_moe(x)
    out, i2, w2 = dev_forward(torch, k3x, layer, x, bf16=bf16)
    assert np.array_equal(i2, idx)
    np.testing.assert_allclose(w2, wt, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2={err:.3e}")
    assert err < TOL


def test_full_repeated_token_columns(torch, k3x, full_normal):
    """Eight copies of one token in a T = 8 call: every column goes through the same
    products and the same part sums, so the eight outputs are equal bit for bit, within
    the parity bar of the single-token call, and a second identical call gives the same
    bits (the down products' parts are added in a fixed order)."""
    say("case: full-size T=8 call of one token repeated, columns and repeat bitwise")
    L, layer = full_normal
    x1 = L.x(1, bf16=True, stream_sub=11)
    x = np.repeat(x1, 8, axis=0)
    out, idx, _ = dev_forward(torch, k3x, layer, x, bf16=True)
    for t in range(1, 8):
        assert np.array_equal(idx[t], idx[0])
        assert np.array_equal(out[t].view(np.uint32), out[0].view(np.uint32)), t
    out2, _, _ = dev_forward(torch, k3x, layer, x, bf16=True)
    assert np.array_equal(out2.view(np.uint32), out.view(np.uint32))
    o1, i1, _ = dev_forward(torch, k3x, layer, x1, bf16=True)
    assert np.array_equal(i1[0], idx[0])
    err = synth.rel_l2(out[:1], o1)
    say(f"  rel_l2 against the single-token call {err:.3e}")
    assert err < TOL
