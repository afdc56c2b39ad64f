"""The oracle of the opt-in MXFP8-activation prefill mode (oracle/k3x_oracle.c, section
"MXFP8-activation prefill mode"), pinned on the CPU.

The mode has no reference counterpart, so its oracle is pinned against what the
definition fixes rather than against reference outputs:
  - E4M3 round-to-nearest-even against a brute-force nearest search over every finite
    E4M3 value (ties to the even code), over all exponents, halfway points and the
    subnormal range;
  - E4M3 decoding against the format's closed form;
  - the block scale: the least X with max|v| <= 448 * 2^X (checked both ways), the
    clamp, and a zero block;
  - the MXFP4 x MXFP8 product against dequantise-then-float64-dot;
  - the identity on activations MXFP8 holds exactly: the product then equals the exact
    path's ko_matmul_mxfp4 on the unquantised row;
  - the whole layer against a numpy composition of the pinned pieces (top-k order,
    routing weight folded in before the second quantisation, shared expert unchanged),
    and its distance from the exact layer (a few percent, as E4M3's 3 mantissa bits give).
"""
import ctypes as C

import numpy as np
import pytest

import synth
from oracle_lib import F32P, U8P, oracle, ptr


def e4m3_table():
    """Every code 0..255 with its value (NaN for 0x7F / 0xFF), by the format's definition."""
    vals = np.empty(256, np.float64)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m * 2.0 ** -9
        else:
            v = (1 + m / 8) * 2.0 ** (e - 7)
        vals[c] = -v if s else v
    return vals


def brute_rne(v, table):
    """Nearest finite E4M3 value to v (|v| <= 448); a tie goes to the even code."""
    fin = np.isfinite(table)
    codes = np.arange(256)[fin]
    vals = table[fin]
    d = np.abs(vals[None, :] - v[:, None])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    out = np.empty(v.shape[0], np.int64)
    for i in range(v.shape[0]):
        cs = codes[cand[i]]
        # +0 and -0 are both nearest to 0: the sign follows v
        if vals[cand[i]].max() == 0.0:
            out[i] = 0x80 if np.signbit(v[i]) else 0
            continue
        ev = cs[(cs & 1) == 0]
        out[i] = ev[0] if len(ev) else cs[0]
    return out


def rne(v):
    lib = oracle()
    return np.array([lib.ko_e4m3_rne(float(x)) for x in v], np.int64)


def test_e4m3_decode_closed_form():
    lib = oracle()
    t = e4m3_table()
    for c in range(256):
        got = lib.ko_e4m3(c)
        if np.isnan(t[c]):
            assert np.isnan(got)
        else:
            assert got == np.float32(t[c]), c
    assert lib.ko_e4m3(0x7E) == 448.0 and lib.ko_e4m3(0x01) == 2.0 ** -9


def test_e4m3_rne_brute_force():
    t = e4m3_table()
    fin = t[np.isfinite(t)]
    pos = np.unique(np.abs(fin))
    mids = (pos[1:] + pos[:-1]) / 2                      # exact halfway points
    rng = np.random.default_rng(0)
    rnd = np.concatenate([
        rng.uniform(-448, 448, 4000),
        np.ldexp(rng.uniform(1, 2, 4000), rng.integers(-14, 9, 4000)) * rng.choice([-1, 1], 4000),
    ])
    near = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, 1000)])
    v = np.concatenate([pos, -pos, mids, -mids, near, -near, rnd]).astype(np.float32)
    v = v[np.abs(v) <= 448]
    got = rne(v)
    want = brute_rne(v.astype(np.float64), t)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (v[bad[:5]], got[bad[:5]], want[bad[:5]])


def test_e4m3_rne_teeth():
    """Round-half-away-from-zero (a plausible slip) differs at the halfway points."""
    t = e4m3_table()
    pos = np.unique(np.abs(t[np.isfinite(t)]))
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    got = rne(mids)
    away = np.array([int(np.argmin(np.abs(t[:0x7F] - m) - 1e-12 * (t[:0x7F] > m)))
                     for m in mids.astype(np.float64)])
    assert (got != away).any()


def scale_of(v):
    return oracle().ko_mx8_scale(ptr(np.ascontiguousarray(v, np.float32), F32P), len(v))


def test_block_scale_is_least_exponent():
    rng = np.random.default_rng(1)
    for _ in range(3000):
        v = (rng.standard_normal(32) * 2.0 ** rng.integers(-60, 60)).astype(np.float32)
        X = scale_of(v) - 127
        amax = float(np.abs(v).max())
        assert amax <= 448 * 2.0 ** X
        assert X == -127 or amax > 448 * 2.0 ** (X - 1)
    assert scale_of(np.zeros(32)) == 0
    v = np.zeros(32, np.float32)
    v[3] = 448.0
    assert scale_of(v) == 127                       # 448 fits at X = 0
    v[3] = np.nextafter(np.float32(448), np.float32(1000))
    assert scale_of(v) == 128
    v[3] = 1e-40                                    # subnormal: clamped to X = -127
    assert scale_of(v) == 0
    v[3] = np.float32(3e38)
    assert scale_of(v) == 127 + 120
    v[5] = np.inf                                   # non-finite elements do not count
    assert scale_of(v) == 127 + 120


def quant(x):
    n = x.shape[0]
    c = np.empty(n, np.uint8)
    s = np.empty(n // 32, np.uint8)
    oracle().ko_mx8_quant(ptr(c, U8P), ptr(s, U8P), ptr(np.ascontiguousarray(x, np.float32), F32P), n)
    return c, s


def dequant(c, s):
    y = np.empty(c.shape[0], np.float64)
    oracle().ko_mx8_dequant(y.ctypes.data_as(C.POINTER(C.c_double)), ptr(c, U8P), ptr(s, U8P),
                            c.shape[0])
    return y


def test_quant_roundtrip_error_bound():
    """Each element is within half an E4M3 step of its block's grid: |q - v| <= 2^-4 |v|
    for normal elements, <= 2^-10 * 2^X in the subnormal range; NaN for non-finite."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(32 * 200) * np.repeat(2.0 ** rng.integers(-20, 20, 200), 32)).astype(np.float32)
    x[7] = np.inf
    x[40] = -np.nan
    c, s = quant(x)
    q = dequant(c, s)
    assert c[7] == 0x7F and c[40] == 0xFF and np.isnan(q[7]) and np.isnan(q[40])
    ok = np.isfinite(x)
    X = np.repeat(s.astype(np.int64) - 127, 32)
    err = np.abs(q - x.astype(np.float64))
    bound = np.maximum(2.0 ** -4 * np.abs(x.astype(np.float64)), 2.0 ** (X - 10))
    assert np.all(err[ok] <= bound[ok] * (1 + 1e-12))


def weights(rng, rows, n, lo=118, hi=130):
    p = rng.integers(0, 256, (rows, n // 2), dtype=np.uint8)
    s = rng.integers(lo, hi, (rows, n // 32), dtype=np.uint8)
    return p, s


def wdeq(p, s):
    y = np.empty((p.shape[0], p.shape[1] * 2), np.float32)
    oracle().ko_mxfp4_dequant(ptr(y, F32P), ptr(p, U8P), ptr(s, U8P), p.shape[0], p.shape[1], 32)
    return y


def mx_mm(c, s, p, ws):
    rows, n = p.shape[0], c.shape[0]
    y = np.empty(rows, np.float32)
    oracle().ko_matmul_mx(ptr(y, F32P), ptr(c, U8P), ptr(s, U8P), ptr(p, U8P), ptr(ws, U8P), n, rows)
    return y


def test_product_against_float64_dot():
    rng = np.random.default_rng(3)
    rows, n = 64, 1024
    p, ws = weights(rng, rows, n)
    x = rng.standard_normal(n).astype(np.float32)
    c, s = quant(x)
    y = mx_mm(c, s, p, ws)
    want = (wdeq(p, ws).astype(np.float64) @ dequant(c, s)).astype(np.float32)
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-30)


def test_identity_on_representable_rows():
    """Integers in [-15, 15] with a 15 in every block are MXFP8 exactly (X = -4): the
    product equals the exact path's ko_matmul_mxfp4 on the same row, to the rounding of
    the latter's sixteen-chain double sum."""
    rng = np.random.default_rng(4)
    rows, n = 64, 1024
    p, ws = weights(rng, rows, n)
    x = rng.integers(-15, 16, n).astype(np.float32)
    x[::32] = 15.0
    c, s = quant(x)
    assert np.array_equal(dequant(c, s), x.astype(np.float64))
    y = mx_mm(c, s, p, ws)
    ye = np.empty(rows, np.float32)
    oracle().ko_matmul_mxfp4(ptr(ye, F32P), ptr(x, F32P), ptr(p, U8P), ptr(ws, U8P), n, rows, 32)
    np.testing.assert_allclose(y, ye, rtol=1e-6)


def numpy_layer_mx(L, x):
    """The MXFP8-activation layer composed in numpy from the pinned pieces."""
    out_e, idx, wt, _ = L.oracle_moe(x)            # routing and the exact layer
    T, H = x.shape
    I = L.I
    out = np.empty_like(x)
    for t in range(T):
        zc, zs = quant(x[t])
        acc = np.zeros(H, np.float32)
        for j in range(L.K):
            d = L.expert(int(idx[t, j]))
            g = mx_mm(zc, zs, d["p1"], d["s1"])
            u = mx_mm(zc, zs, d["p3"], d["s3"])
            gu = np.concatenate([g, u]).astype(np.float32)
            act = np.empty(I, np.float32)
            oracle().ko_situ_glu(ptr(act, F32P), ptr(gu, F32P), I, np.float32(L.situ_b1),
                                 np.float32(L.situ_b2))
            h = (np.float32(wt[t, j]) * act).astype(np.float32)
            hc, hs = quant(h)
            acc = (acc + mx_mm(hc, hs, d["p2"], d["s2"])).astype(np.float32)
        out[t] = acc
    return out, idx, out_e


def test_layer_against_numpy_composition():
    L = synth.tiny(seed=5, n_shared=0)
    x = L.x(5, bf16=False)
    o, idx, wt, drops = L.oracle_moe_mx(x)
    want, widx, exact = numpy_layer_mx(L, x)
    assert drops == 0 and np.array_equal(idx, widx)
    assert np.array_equal(o.view(np.uint32), want.view(np.uint32))
    err = synth.rel_l2(o, exact)
    assert 1e-3 < err < 5e-2, err


def test_layer_shared_expert_and_latent_unquantised():
    """The shared expert is the exact path's: with one, the MX layer minus the same layer
    without it equals the exact layers' difference.  A LatentMoE layer runs (z quantised
    at the latent width) and stays within a few percent of the exact layer."""
    L0 = synth.tiny(seed=6, n_shared=0)
    L1 = synth.tiny(seed=6, n_shared=1)
    x = L1.x(3, bf16=False)
    m0, _, _, _ = L0.oracle_moe_mx(x)
    m1, _, _, _ = L1.oracle_moe_mx(x)
    e0, _, _, _ = L0.oracle_moe(x)
    e1, _, _, _ = L1.oracle_moe(x)
    # (routed + shared) - routed recovers the shared row up to the float rounding of
    # the sums, a few ulps of the routed magnitude
    tol = 4 * float(np.spacing(np.float32(max(np.abs(m1).max(), np.abs(e1).max()))))
    np.testing.assert_allclose(m1 - m0, e1 - e0, rtol=0, atol=tol)
    La = synth.tiny_latent(seed=0)
    xa = La.x(3, bf16=False)
    ma, ia, _, _ = La.oracle_moe_mx(xa)
    ea, ie, _, _ = La.oracle_moe(xa)
    assert np.array_equal(ia, ie)
    assert synth.rel_l2(ma, ea) < 5e-2
