"""MXFP4 dequantisation on the device, bit for bit (k3_mxfp4_dequant, k3_ops.c:3778-3808;
the reference's KAT t_mxfp4, tests/unit/test_ops.c:1212-1270).

A layer's expert matrices are read back through the product kernels' own conversion
(k3x_moe_layer_dequant: dq8 for scale bytes 1..252, dq8_exact when the layer holds any
other byte) and compared with
  - the reference's fixture tests/fixtures/mxfp4.json (64 rows x 3584 elements of the
    released checkpoint's bytes, layer 1 expert 0 w1, with their exact floats), placed in
    rows 0..63 of an expert's gate matrix at the fixture's own width, and
  - the oracle's ko_mxfp4_dequant on every row, including rows whose scale bytes cycle
    through every value: 0 (2^-127), 253 and 254 (products that overflow to infinity), 255
    (zero);
exactly (the float bits, signs of zero and infinities included).  A layer forward with
scale bytes 0, 253, 254 and 255 is then checked against the oracle.
"""
import os

import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, say
from oracle_lib import F32P, U8P, oracle, ptr

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-3


def oracle_dequant(p, s):
    y = np.empty((p.shape[0], p.shape[1] * 2), np.float32)
    oracle().ko_mxfp4_dequant(ptr(y, F32P), ptr(np.ascontiguousarray(p), U8P),
                              ptr(np.ascontiguousarray(s), U8P), p.shape[0], p.shape[1], 32)
    return y


def kat_layer(k3x, scale_cycle):
    """hidden 3584 (the fixture's width), 2 experts top-1, I 128, no shared expert; expert
    0's gate rows 0..63 hold the fixture's bytes, rows 64..127 random codes with scale
    bytes cycling over scale_cycle."""
    g = np.load(os.path.join(GOLD, "ref_mxfp4.npz"))
    L = synth.Layer(H=3584, E=2, K=1, I=128, n_shared=0, seed=5)
    d = L.expert(0)
    rng = np.random.default_rng(11)
    d["p1"][:64] = g["packed"]
    d["s1"][:64] = g["scales"]
    d["p1"][64:] = rng.integers(0, 256, d["p1"][64:].shape, dtype=np.uint8)
    n = d["s1"][64:].size
    d["s1"][64:] = np.resize(np.asarray(scale_cycle, np.uint8), n).reshape(d["s1"][64:].shape)
    return L, g


@pytest.mark.parametrize("path", ["fast", "exact"])
def test_dequant_real_checkpoint_bytes(torch, k3x, path):
    """fast: scale bytes 1..252 only, so the layer's kernels take the v_cvt_scalef32
    conversion; exact: every byte 0..255 present, so they take the exact path."""
    cyc = np.arange(1, 253) if path == "fast" else np.arange(0, 256)
    say(f"case: device dequant of the released checkpoint bytes ({path} path)")
    L, g = kat_layer(k3x, cyc)
    layer = bank_layer(k3x, L)
    got = layer.dequant(0, 0)
    d = L.expert(0)
    want = oracle_dequant(d["p1"], d["s1"])
    assert np.array_equal(got[:64].view(np.uint32), g["expected"].view(np.uint32)), \
        "device dequant differs from the reference fixture's exact floats"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if path == "exact":
        assert np.isinf(got).any() and (got[64:] == 0).any()
    for m, (pk, sk) in ((1, ("p3", "s3")), (2, ("p2", "s2"))):
        assert np.array_equal(layer.dequant(0, m).view(np.uint32),
                              oracle_dequant(d[pk], d[sk]).view(np.uint32))
    layer.close()


def test_forward_with_special_scale_bytes(torch, k3x):
    """Scale bytes 0 (2^-127) and 255 (zero) in gate, up and down; 253 and 254 in down on
    groups whose codes are 0 or +-0.5, so the weights (+-2^125, +-2^126) are finite and the
    outputs stay finite but huge on the rows they reach.  Against the oracle (the layer
    takes the exact dequantisation path for all three matrices)."""
    say("case: tiny layer forward with scale bytes 0, 253, 254, 255")
    # small gate/up scales (2^-13 .. 2^-9) keep the activations near 1e-4, so a single
    # 2^126 weight times one of them stays far below the float range
    L = synth.tiny(seed=7, scale_lo=114, scale_hi=118)
    for e in range(L.E):
        d = L.expert(e)
        for sk in ("s1", "s3", "s2"):
            f = d[sk].reshape(-1)
            f[::7] = 0
            f[3::11] = 255
        s2 = d["s2"]
        for (r, gi, b) in ((e % 16, 1, 253), ((e * 5) % 256, 3, 254)):
            s2[r, gi] = b
            row = d["p2"][r, gi * 16:(gi + 1) * 16]
            row[:] = np.random.default_rng(e).choice(
                np.array([0x00, 0x01, 0x08, 0x09, 0x10, 0x11, 0x18, 0x19, 0x80, 0x81, 0x88,
                          0x89, 0x90, 0x91, 0x98, 0x99], np.uint8), 16)
    layer = bank_layer(k3x, L)
    x = L.x(5, bf16=False, stream_sub=3)
    o, idx, _, _ = L.oracle_moe(x)
    assert np.isfinite(o).all() and np.abs(o).max() > 1e30
    out, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx)
    err = synth.rel_l2(out, o)
    say(f"  max |out| {np.abs(o).max():.3e}, rel_l2={err:.3e}")
    assert err < TOL
    layer.close()
