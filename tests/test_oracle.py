"""Pins the oracle (oracle/k3x_oracle.c) before device results are checked against it.

Three kinds of evidence, per function:
  * the reference's own fixtures (tests/golden/ref_*.npz, converted from the
    reference's tests/fixtures JSON by tests/golden/make_golden.py);
  * bit-for-bit agreement with the COMPILED reference (oracle/_ref), on data built so
    that any other summation order changes the bits (skipped where it is not built);
  * closed forms and brute force on inputs where the exact answer is known.
Each order-sensitive check is paired with a "teeth" check showing that a plausible
wrong order fails on the same data.
"""
import ctypes as C
import os

import numpy as np
import pytest

import synth
from oracle_lib import F32P, I32P, KoExpert, U8P, U16P, oracle, ptr, ref

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def gold(name):
    return np.load(os.path.join(GOLD, name))


def e8m0(b):
    b = np.asarray(b, np.int64)
    with np.errstate(over="ignore"):
        v = np.ldexp(np.float32(1.0), (b - 127).astype(np.int32)).astype(np.float32)
    return np.where(b == 255, np.float32(0), v).astype(np.float32)


def dequant_np(packed, scales, group=32):
    lo = packed & 15
    hi = packed >> 4
    codes = np.stack([lo, hi], -1).reshape(packed.shape[0], -1)
    s = np.repeat(e8m0(scales), group, axis=1)[:, :codes.shape[1]]
    return (E2M1[codes] * s).astype(np.float32)


def mx_gemv(x, p, s, group=32):
    rows, pc = p.shape
    y = np.empty(rows, np.float32)
    rc = oracle().ko_matmul_mxfp4(ptr(y, F32P), ptr(x, F32P), ptr(p, U8P), ptr(s, U8P),
                                  2 * pc, rows, group)
    assert rc == 0
    return y


def bf16_gemv(x, W):
    out, n = W.shape
    y = np.empty(out, np.float32)
    oracle().ko_matmul_bf16(ptr(y, F32P), ptr(x, F32P), ptr(W, U16P), n, out)
    return y


# ------------------------------------------------------------------ MXFP4 decode
def test_mxfp4_fixture_dequant_exact():
    g = gold("ref_mxfp4.npz")
    p, s, exp = g["packed"], g["scales"], g["expected"]
    assert np.array_equal(g["lut"], E2M1)
    y = np.empty(exp.shape, np.float32)
    oracle().ko_mxfp4_dequant(ptr(y, F32P), ptr(p, U8P), ptr(s, U8P), p.shape[0], p.shape[1],
                              int(g["group"]))
    assert np.array_equal(y.view(np.uint32), exp.view(np.uint32))
    # the oracle's tables against the closed form
    for c in range(16):
        assert oracle().ko_e2m1(c) == E2M1[c]
    for b in range(256):
        assert np.float32(oracle().ko_e8m0(b)) == e8m0(b)


def test_mxfp4_fixture_swapped_nibbles_rejected():
    g = gold("ref_mxfp4.npz")
    p, s = g["packed"], g["scales"]
    sw = ((p & 15) << 4) | (p >> 4)
    y = np.empty(g["expected"].shape, np.float32)
    oracle().ko_mxfp4_dequant(ptr(y, F32P), ptr(sw, U8P), ptr(s, U8P), p.shape[0], p.shape[1], 32)
    assert not np.array_equal(y, g["expected"])
    assert np.array_equal(y[0, :64], g["swapped_first64"])


def test_mxfp4_gemv_vs_dequant_dot():
    """Real checkpoint bytes: the fused GEMV within 1e-6 of dequantise-then-dot
    (test_expert.c:227's contract), rows independent."""
    g = gold("ref_mxfp4.npz")
    p, s = g["packed"], g["scales"]
    rng = np.random.default_rng(0)
    x = rng.standard_normal(2 * p.shape[1]).astype(np.float32)
    y = mx_gemv(x, p, s)
    want = g["expected"].astype(np.float64) @ x.astype(np.float64)
    rel = np.abs(y - want) / np.maximum(np.abs(want), 1e-30)
    assert rel.max() < 1e-6


def cancelling(rows, n, rng, big=60):
    """x with +2^big and -2^big at adjacent positions p, p+1 (p = n/2, even) among
    N(0,1) values.  Where the weights at p and p+1 are equal the two cancel exactly,
    and which small terms they swallowed first depends on the summation order."""
    x = rng.standard_normal(n).astype(np.float32)
    p = (n // 2) & ~1
    x[p] = np.float32(2.0 ** big)
    x[p + 1] = -np.float32(2.0 ** big)
    return x


def cancelling_codes(p_bytes, n):
    """Make every row's codes at columns n/2 and n/2+1 both 1.0 (code 2)."""
    q = p_bytes.copy()
    q[:, ((n // 2) & ~1) // 2] = 0x22
    return q


@pytest.mark.parametrize("seed", [0, 1])
def test_mxfp4_gemv_bitwise_vs_reference(seed, ref_lib):
    rng = np.random.default_rng(seed)
    rows, n = 96, 3584
    p = rng.integers(0, 256, (rows, n // 2), dtype=np.uint8)
    s = rng.integers(118, 130, (rows, n // 32), dtype=np.uint8)
    s[3, 5] = 255
    s[7, 0] = 0
    s[8, 1] = 1
    s[9, 2] = 254
    s[10, 3] = 253
    p = cancelling_codes(p, n)
    for x in (rng.standard_normal(n).astype(np.float32), cancelling(rows, n, rng)):
        y = mx_gemv(x, p, s)
        r = np.empty(rows, np.float32)
        ref_lib.k3_matmul_mxfp4(ptr(r, F32P), ptr(x, F32P), ptr(p, U8P), ptr(s, U8P), n, rows, 32)
        assert np.array_equal(y.view(np.uint32), r.view(np.uint32))


def test_mxfp4_gemv_order_teeth():
    """On cancelling data a sequential double sum (a plausible wrong order) differs."""
    rng = np.random.default_rng(5)
    rows, n = 64, 3584
    p = cancelling_codes(rng.integers(0, 256, (rows, n // 2), dtype=np.uint8), n)
    s = rng.integers(120, 126, (rows, n // 32), dtype=np.uint8)
    x = cancelling(rows, n, rng)
    y = mx_gemv(x, p, s)
    assert np.abs(y).max() < 1e6                 # the big pair cancelled
    W = dequant_np(p, s).astype(np.float64)
    seq = np.zeros(rows)
    for i in range(n):
        seq = seq + W[:, i] * np.float64(x[i])
    assert not np.array_equal(y, seq.astype(np.float32))


def test_mxfp4_scale255_skips_group():
    rng = np.random.default_rng(3)
    p = rng.integers(0, 256, (4, 64), dtype=np.uint8)
    s = np.full((4, 4), 124, np.uint8)
    s[1, 2] = 255
    x = rng.standard_normal(128).astype(np.float32)
    y = mx_gemv(x, p, s)
    W = dequant_np(p, s).astype(np.float64)     # group of byte 255 dequantises to 0
    assert np.allclose(y, W @ x, rtol=1e-6, atol=1e-6)


def test_mxfp4_rejects_bad_shapes():
    y = np.empty(1, np.float32)
    x = np.zeros(34, np.float32)
    p = np.zeros(17, np.uint8)
    s = np.zeros(2, np.uint8)
    assert oracle().ko_matmul_mxfp4(ptr(y, F32P), ptr(x, F32P), ptr(p, U8P), ptr(s, U8P), 33, 1, 32) == -1
    assert oracle().ko_matmul_mxfp4(ptr(y, F32P), ptr(x, F32P), ptr(p, U8P), ptr(s, U8P), 34, 1, 24) == -1


# ------------------------------------------------------------------ bf16 GEMV
def test_bf16_gemv_bitwise_vs_reference(ref_lib):
    rng = np.random.default_rng(11)
    out, n = 70, 2051               # odd sizes: tail and odd row
    W = synth.f32_to_bf16(rng.standard_normal((out, n)).astype(np.float32))
    W[:, (n // 2) & ~1] = W[:, ((n // 2) & ~1) + 1] = 0x3F80
    for x in (rng.standard_normal(n).astype(np.float32), cancelling(out, n, rng, big=40)):
        y = bf16_gemv(x, W)
        r = np.empty(out, np.float32)
        ref_lib.k3_matmul_bf16(ptr(r, F32P), ptr(x, F32P), ptr(W, U16P), n, out)
        assert np.array_equal(y.view(np.uint32), r.view(np.uint32))


def test_bf16_gemv_nan_canonical():
    W = np.zeros((2, 32), np.uint16)
    W[0, 3] = 0xFFC1                # a NaN with payload and sign
    x = np.ones(32, np.float32)
    y = bf16_gemv(x, W)
    assert y.view(np.uint32)[0] == 0x7FC00000
    assert y[1] == 0.0


def test_bf16_gemv_exact_on_integers():
    """Small integers: every order gives the exact sum."""
    rng = np.random.default_rng(2)
    Wf = rng.integers(-8, 9, (33, 515)).astype(np.float32)
    x = rng.integers(-8, 9, 515).astype(np.float32)
    y = bf16_gemv(x, synth.f32_to_bf16(Wf))
    assert np.array_equal(y, (Wf.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))


# ------------------------------------------------------------------ router
def route(x, W, b, K, renorm=1, scale=1.0):
    E, H = W.shape
    idx = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    oracle().ko_router(ptr(idx, I32P), ptr(w, F32P), ptr(x, F32P), ptr(W, F32P),
                       ptr(b, F32P) if b is not None else None, H, E, K, renorm, scale)
    return idx, w


def test_router_reference_fixture():
    g = gold("ref_router.npz")
    W, b, X = g["gate"], g["bias"], g["x"]
    K = int(g["top_k"])
    for t in range(X.shape[0]):
        idx, w = route(np.ascontiguousarray(X[t]), W, b, K)
        assert set(idx.tolist()) == set(g["topk_idx"][t].tolist())
        order = np.argsort(g["topk_idx"][t])
        mine = np.argsort(idx)
        np.testing.assert_allclose(w[mine], g["topk_weight"][t][order], rtol=1e-4, atol=1e-5)
    assert int(g["rows_bias_changed"]) == 5


def test_router_bitwise_vs_reference(ref_lib):
    rng = np.random.default_rng(7)
    for E, H, K in ((16, 256, 4), (384, 7168, 8), (40, 128, 16)):
        W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        b = (rng.standard_normal(E) * 0.1).astype(np.float32)
        x = rng.standard_normal(H).astype(np.float32)
        i1, w1 = route(x, W, b, K, 1, 2.5)
        i2 = np.empty(K, np.int32)
        w2 = np.empty(K, np.float32)
        ref_lib.k3_router(ptr(i2, I32P), ptr(w2, F32P), ptr(x, F32P), ptr(W, F32P), ptr(b, F32P),
                          H, E, K, 1, 2.5)
        assert np.array_equal(i1, i2) and np.array_equal(w1.view(np.uint32), w2.view(np.uint32))


def test_router_bruteforce_ties_lower_index():
    """Exactly representable logits (any order sums them exactly) with deliberate ties:
    selection must be the first K of the order (-choice, index)."""
    rng = np.random.default_rng(9)
    E, H, K = 48, 64, 8
    W = rng.integers(-4, 5, (E, H)).astype(np.float32) / 8
    W[10] = W[3]
    W[20] = W[3]
    W[33] = W[5]
    x = rng.integers(-4, 5, H).astype(np.float32) / 4
    logit = (W.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    assert logit[10] == logit[3] == logit[20]
    for bias in (None, np.zeros(E, np.float32)):
        idx, w = route(x, W, bias, K, renorm=0)
        score = (1.0 / (1.0 + np.exp(-logit.astype(np.float64)))).astype(np.float32)
        want = np.lexsort((np.arange(E), -score))[:K]
        assert np.array_equal(idx, want)
        np.testing.assert_allclose(w, score[want], rtol=2e-7)


def test_router_renorm_and_scale():
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((64, 128)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(64) * 0.1).astype(np.float32)
    x = rng.standard_normal(128).astype(np.float32)
    idx, w = route(x, W, b, 6, renorm=1, scale=2.5)
    assert abs(float(w.astype(np.float64).sum()) - 2.5) < 1e-5
    idx0, w0 = route(x, W, b, 6, renorm=0, scale=1.0)
    assert np.array_equal(idx, idx0)
    logit = W.astype(np.float64) @ x.astype(np.float64)
    score = 1 / (1 + np.exp(-logit))
    np.testing.assert_allclose(w0, score[idx0], rtol=1e-6)       # UNBIASED scores


# ------------------------------------------------------------------ SiTU / RMSNorm
def test_situ_reference_fixture():
    g = gold("ref_situ_glu.npz")
    X = g["x"]
    n = X.shape[1] // 2
    for t in range(X.shape[0]):
        x = np.ascontiguousarray(X[t])
        y = np.empty(n, np.float32)
        oracle().ko_situ_glu(ptr(y, F32P), ptr(x, F32P), n, float(g["beta"]), float(g["linear_beta"]))
        np.testing.assert_allclose(y, g["out"][t], rtol=1e-4, atol=1e-5)


def test_situ_swiglu_limit():
    rng = np.random.default_rng(1)
    n = 4096
    x = (rng.standard_normal(2 * n) * 8).astype(np.float32)
    y = np.empty(n, np.float32)
    oracle().ko_situ_glu(ptr(y, F32P), ptr(x, F32P), n, 2.0 ** 64, 2.0 ** 64)
    g, u = x[:n].astype(np.float64), x[n:].astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-30)


def test_rmsnorm_reference_fixture():
    g = gold("ref_rmsnorm.npz")
    X = g["x"]
    for t in range(X.shape[0]):
        x = np.ascontiguousarray(X[t])
        y = np.empty_like(x)
        oracle().ko_rmsnorm(ptr(y, F32P), ptr(x, F32P), ptr(g["w"], F32P), x.size, float(g["eps"]))
        np.testing.assert_allclose(y, g["out"][t], rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ whole layer
def ref_bank(L):
    bank = (KoExpert * L.E)()
    keep = []
    for e in range(L.E):
        d = L.expert(e)
        keep.append(d)
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            setattr(bank[e], k, d[k].ctypes.data_as(U8P))
    return bank, keep


def ref_moe(ref_lib, L, x, prefill, fail=None):
    bank, keep = ref_bank(L)
    T = x.shape[0]
    out = np.empty_like(x)
    idx = np.empty(L.K, np.int32)
    wt = np.empty(L.K, np.float32)
    gets = C.c_long(0)
    fa = None
    if fail is not None:
        fa = np.zeros(L.E, np.int32)
        fa[list(fail)] = 1
    drops = ref_lib.refdrv_moe(ptr(out, F32P), ptr(x, F32P), T, L.H, L.E, L.K, L.I, L.n_shared,
                               L.routed_scale, L.renorm, ptr(L.gate, F32P), ptr(L.bias, F32P),
                               bank, ptr(fa, I32P) if fa is not None else None,
                               ptr(L.sh1, U16P), ptr(L.sh3, U16P), ptr(L.sh2, U16P),
                               1 if prefill else 0, ptr(idx, I32P), ptr(wt, F32P), C.byref(gets))
    return out, idx, wt, drops, gets.value


@pytest.mark.parametrize("seed", [0, 3])
def test_moe_bitwise_vs_reference_tiny(seed, ref_lib):
    L = synth.tiny(seed=seed)
    x = L.x(6, bf16=False)
    o, idx, wt, d = L.oracle_moe(x)
    r, ri, rw, rd, _ = ref_moe(ref_lib, L, x, prefill=False)
    assert d == 0 and rd == 0
    assert np.array_equal(o.view(np.uint32), r.view(np.uint32))
    assert np.array_equal(idx[-1], ri) and np.array_equal(wt[-1].view(np.uint32), rw.view(np.uint32))


def test_moe_prefill_dedup_bitwise(ref_lib):
    """T = 130 over 64-token sub-chunks, top-16 of 40: batched prefill is bitwise equal
    to per-token and to the reference's k3_moe_prefill; get() runs once per unique
    expert per sub-chunk (test_ops.c:891-1014's gate, on this layer)."""
    L = synth.Layer(H=256, E=40, K=16, I=128, seed=4, scale_lo=121, scale_hi=124)
    x = L.x(130, bf16=False)
    op, pidx, pwt, pd, ng = L.oracle_moe(x, prefill=True)
    o, idx, wt, d = L.oracle_moe(x)
    assert np.array_equal(op.view(np.uint32), o.view(np.uint32))
    assert np.array_equal(pidx, idx)
    want_gets = sum(len(np.unique(idx[t0:t0 + 64])) for t0 in range(0, 130, 64))
    assert ng == want_gets
    r, ri, rw, rd, rg = ref_moe(ref_lib, L, x, prefill=True)
    assert np.array_equal(op.view(np.uint32), r.view(np.uint32))
    assert rg == want_gets


def k2_direct(lib, fn, L, x):
    """One of the harness's K2 compositions of the reference's kernels (refdrv_k2_tokens,
    refdrv_k2_prefill) over the rows of x; routing of every row returned."""
    bank, keep = ref_bank(L)
    T = x.shape[0]
    out = np.empty_like(x)
    idx = np.empty((T, L.K), np.int32)
    wt = np.empty((T, L.K), np.float32)
    rc = getattr(lib, fn)(ptr(out, F32P), ptr(x, F32P), T, L.H, L.E, L.K, L.I,
                          L.I * L.n_shared, L.routed_scale, L.renorm, ptr(L.gate, F32P),
                          ptr(L.bias, F32P), bank, ptr(L.sh1, U16P), ptr(L.sh3, U16P),
                          ptr(L.sh2, U16P), ptr(idx, I32P), ptr(wt, F32P))
    assert rc == 0
    return out, idx, wt


def test_ref_k2_compositions_bitwise(ref_lib):
    """The compositions of the reference's own kernels that the CPU baselines time
    (refdrv_k2_tokens: a decode token; refdrv_k2_prefill: a prefill chunk, sub-chunks
    of 64, unique experts expert-major, the batched shared products) give the bits of
    the reference's k3_moe and k3_moe_prefill themselves: 130 tokens over three
    sub-chunks, top-16 of 40, and every token's routing is the oracle's."""
    L = synth.Layer(H=256, E=40, K=16, I=128, seed=4, scale_lo=121, scale_hi=124)
    x = L.x(130, bf16=False)
    rp = ref_moe(ref_lib, L, x, prefill=True)[0]
    rd = ref_moe(ref_lib, L, x, prefill=False)[0]
    p, pidx, pwt = k2_direct(ref_lib, "refdrv_k2_prefill", L, x)
    d, didx, dwt = k2_direct(ref_lib, "refdrv_k2_tokens", L, x)
    assert np.array_equal(p.view(np.uint32), rp.view(np.uint32))
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    _, oidx, owt, _ = L.oracle_moe(x)
    for i, w in ((pidx, pwt), (didx, dwt)):
        assert np.array_equal(i, oidx) and np.array_equal(w.view(np.uint32), owt.view(np.uint32))


def test_ref_k2_norm_layer_bitwise(ref_lib):
    """refdrv_k2_norm_layer, the step the stack's CPU baseline times (h = h +
    MoE(RMSNorm(h)), the reference's k3_rmsnorm and k3_moe work), against the oracle's
    RMSNorm, whole layer and float residual add: three layers in turn, five rows."""
    layers = [synth.tiny(seed=10 + l, layer=l) for l in range(3)]
    h = layers[0].x(5, bf16=False, stream_sub=7)
    hr = h.copy()
    for L in layers:
        w = synth.normal_f32(L.H, synth.key(L.seed, L.layer, synth.S_NORM), 1.0, 0.1)
        hin = np.empty_like(h)
        for t in range(h.shape[0]):
            oracle().ko_rmsnorm(ptr(hin[t], F32P), ptr(np.ascontiguousarray(h[t]), F32P),
                                ptr(w, F32P), L.H, 1e-5)
        h = h + L.oracle_moe(hin)[0]
        bank, keep = ref_bank(L)
        idx = np.empty((h.shape[0], L.K), np.int32)
        wt = np.empty((h.shape[0], L.K), np.float32)
        rc = ref_lib.refdrv_k2_norm_layer(ptr(hr, F32P), hr.shape[0], ptr(w, F32P), 1e-5, L.H,
                                          L.E, L.K, L.I, L.I * L.n_shared, L.routed_scale,
                                          L.renorm, ptr(L.gate, F32P), ptr(L.bias, F32P), bank,
                                          ptr(L.sh1, U16P), ptr(L.sh3, U16P), ptr(L.sh2, U16P),
                                          ptr(idx, I32P), ptr(wt, F32P))
        assert rc == 0
        assert np.array_equal(h.view(np.uint32), hr.view(np.uint32))


def test_moe_combine_order_teeth():
    """Summing a token's expert outputs in first-seen (fetch) order instead of top-k
    order changes the floats at top-16 (the slip k3_ops.c:2113-2118 warns about)."""
    L = synth.Layer(H=256, E=40, K=16, I=128, seed=4, scale_lo=121, scale_hi=124, n_shared=0)
    x = L.x(64, bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    cfg = L.ko_cfg()
    diffs = 0
    for t in range(64):
        contribs = []
        for j in range(L.K):
            d = L.expert(int(idx[t, j]))
            gu = np.concatenate([mx_gemv(x[t], d["p1"], d["s1"]), mx_gemv(x[t], d["p3"], d["s3"])])
            act = np.empty(L.I, np.float32)
            oracle().ko_situ_glu(ptr(act, F32P), ptr(gu, F32P), L.I, cfg.situ_b1, cfg.situ_b2)
            contribs.append((wt[t, j], mx_gemv(act, d["p2"], d["s2"])))
        acc = np.zeros(L.H, np.float32)
        for w, c in contribs:
            acc = (acc + np.float32(w) * c).astype(np.float32)
        assert np.array_equal(acc.view(np.uint32), o[t].view(np.uint32))   # top-k order
        acc2 = np.zeros(L.H, np.float32)
        for j in np.argsort(idx[t]):
            acc2 = (acc2 + np.float32(contribs[j][0]) * contribs[j][1]).astype(np.float32)
        diffs += not np.array_equal(acc2, o[t])
    assert diffs > 0


def test_moe_drop_counted_and_skipped(ref_lib):
    L = synth.tiny(seed=1)
    x = L.x(3, bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    victim = int(idx[0, 1])
    od, idxd, wtd, drops = L.oracle_moe(x, fail={victim})
    assert drops == int((idx == victim).sum())
    assert not np.array_equal(od[0], o[0])
    r, _, _, rd, _ = ref_moe(ref_lib, L, x, prefill=False, fail={victim})
    assert rd == drops
    assert np.array_equal(od.view(np.uint32), r.view(np.uint32))


def test_golden_k2_tiny():
    g = gold("k2_tiny.npz")
    L = synth.tiny(seed=int(g["seed"]))
    x = L.x(int(g["T"]), bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    assert np.array_equal(idx, g["idx"])
    assert np.array_equal(wt.view(np.uint32), g["wt"].view(np.uint32))
    assert np.array_equal(o.view(np.uint32), g["out"].view(np.uint32))


def fnv1a(a):
    h = 0xCBF29CE484222325
    for b in np.ascontiguousarray(a).view(np.uint8).tobytes():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


@pytest.mark.parametrize("name,kw,sub", [("normal", {}, 0), ("zipf", {"zipf_alpha": 1.0}, 1)])
def test_golden_k2_full(name, kw, sub):
    """Full K2 shape, against vectors the compiled reference produced."""
    g = gold("k2_full.npz")
    L = synth.full(seed=1, **kw)
    x = L.x(2, bf16=True, stream_sub=sub)
    o, idx, wt, _ = L.oracle_moe(x)
    assert np.array_equal(idx, g[name + "_idx"])
    assert np.array_equal(wt.view(np.uint32), g[name + "_wt"].view(np.uint32))
    for t in range(2):
        assert np.array_equal(o[t, ::16].view(np.uint32), g[name + "_out16"][t].view(np.uint32))
        assert fnv1a(o[t]) == int(g[name + "_hash"][t])


def test_generator_reproducible():
    a = synth.normal_f32(1000, synth.key(5, 2, 0, 0))
    b = synth.normal_f32(1000, synth.key(5, 2, 0, 0))
    c = synth.normal_f32(1000, synth.key(5, 3, 0, 0))
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 0.1 and abs(a.std() - 1) < 0.1
    s = synth.scales(100000, synth.key(1, 0, 11, 0), 121, 125)
    assert s.min() == 121 and s.max() == 125
    cd = synth.codes(100000, synth.key(1, 0, 10, 0))
    nib = np.concatenate([cd & 15, cd >> 4])
    assert np.bincount(nib, minlength=16).min() > 100000 * 2 / 16 * 0.9


def test_reference_avx512_build_bitwise():
    """The reference compiled for x86-64-v4 (its AVX-512 paths, k3_ops.c:457, :2752,
    :3134, the build the CPU baseline uses on such hosts) gives the same bits as the
    oracle: the GEMV on cancelling data and the whole tiny layer, decode and prefill."""
    import oracle_lib as ol
    r4 = ol.ref("x86-64-v4")
    if r4 is None:
        pytest.skip("no AVX-512 host, or oracle/_ref not built")
    rng = np.random.default_rng(9)
    rows, n = 96, 3584
    p = cancelling_codes(rng.integers(0, 256, (rows, n // 2), dtype=np.uint8), n)
    s = rng.integers(118, 130, (rows, n // 32), dtype=np.uint8)
    x = cancelling(rows, n, rng)
    y = mx_gemv(x, p, s)
    r = np.empty(rows, np.float32)
    r4.k3_matmul_mxfp4(ptr(r, F32P), ptr(x, F32P), ptr(p, U8P), ptr(s, U8P), n, rows, 32)
    assert np.array_equal(y.view(np.uint32), r.view(np.uint32))
    L = synth.tiny(seed=2)
    xt = L.x(70, bf16=False)
    for prefill in (False, True):
        o, _, _, _ = L.oracle_moe(xt, prefill=prefill)[:4]
        ro, _, _, rd, _ = ref_moe(r4, L, xt, prefill=prefill)
        assert rd == 0 and np.array_equal(o.view(np.uint32), ro.view(np.uint32))


@pytest.mark.parametrize("latent", [False, True])
def test_host_layer_check_bitwise(ref_lib, latent):
    """The host side of the GPU tests' many-token checks (gpu_util.host_layer: the
    compiled reference's prefill over a sample of rows, only the chosen experts
    generated) equals the oracle's whole layer bit for bit, K2 and latent forms, on rows
    taken from over a larger call."""
    from gpu_util import host_layer
    L = synth.tiny_latent(seed=6) if latent else synth.tiny(seed=6)
    x = L.x(150, bf16=True, stream_sub=3)
    o, idx, _, _ = L.oracle_moe(x)
    rows = np.r_[np.arange(0, 150, 2), 149]
    h, what = host_layer(L, x[rows], idx[rows])
    assert "compiled reference" in what
    assert np.array_equal(h.view(np.uint32), o[rows].view(np.uint32))
    assert not L._held
