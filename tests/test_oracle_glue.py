"""Pins the oracle's decoder-layer glue: ko_attn_res against the reference's fixture
attnres.json (tests/golden/ref_attnres.npz) at its op tolerance and bitwise against the
compiled reference's k3_attn_res; one source returns that source; ko_moe_half with no
block residual is one step of ko_stack_step (h += MoE(RMSNorm(h)))."""
import os

import numpy as np
import pytest

import synth
from oracle_lib import F32P, oracle, ptr

HERE = os.path.dirname(os.path.abspath(__file__))


def attn_res(src, fold, eps, fn=None):
    out = np.empty(src.shape[1], np.float32)
    src = np.ascontiguousarray(src, np.float32)
    (fn or oracle().ko_attn_res)(ptr(out, F32P), ptr(src, F32P), ptr(fold, F32P), src.shape[0],
                                 src.shape[1], eps)
    return out


def test_attn_res_reference_fixture():
    g = np.load(os.path.join(HERE, "golden", "ref_attnres.npz"))
    fold = np.ascontiguousarray(g["fold"], np.float32)
    rows, nblk, n = g["blocks"].shape
    assert nblk + 1 == int(g["n_sources"])
    for r in range(rows):
        src = np.concatenate([g["blocks"][r], g["prefix"][r:r + 1]])
        np.testing.assert_allclose(attn_res(src, fold, float(g["eps"])), g["out"][r],
                                   atol=float(g["tol_abs"]), rtol=float(g["tol_rel"]))


def test_attn_res_bitwise_vs_reference(ref_lib):
    rng = np.random.default_rng(0)
    for nsrc, n in ((1, 64), (5, 256), (13, 7168)):
        src = (rng.standard_normal((nsrc, n)) * rng.uniform(0.1, 10, (nsrc, 1))).astype(np.float32)
        fold = rng.standard_normal(n).astype(np.float32)
        a = attn_res(src, fold, 1e-5)
        b = attn_res(src, fold, 1e-5, ref_lib.k3_attn_res)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_attn_res_single_source_is_identity():
    rng = np.random.default_rng(1)
    v = rng.standard_normal((1, 300)).astype(np.float32)
    out = attn_res(v, rng.standard_normal(300).astype(np.float32), 1e-5)
    assert np.array_equal(out, v[0])


def test_moe_half_without_blocks_is_a_stack_step():
    import ctypes as C
    L = synth.tiny(seed=31)
    T, H = 3, L.H
    rng = np.random.default_rng(2)
    pref = L.x(T, bf16=False) * 2
    post = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    fold = rng.standard_normal(H).astype(np.float32)
    cfg = L.ko_cfg()
    w, cb, keep = L._weights()
    h = np.empty_like(pref)
    p = pref.copy()
    oracle().ko_moe_half(ptr(h, F32P), ptr(p, F32P), None, 0, 0, ptr(fold, F32P),
                         ptr(post, F32P), 1e-5, T, C.byref(cfg), C.byref(w))
    want = pref.copy()
    wl = (C.POINTER(type(w)) * 1)(C.pointer(w))
    nl = (F32P * 1)(ptr(post, F32P))
    oracle().ko_stack_step(ptr(want, F32P), T, 1, C.byref(cfg), wl, nl, 1e-5)
    assert np.array_equal(h.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(p.view(np.uint32), want.view(np.uint32))
