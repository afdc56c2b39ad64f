"""Pins the oracle's decoder-layer glue: ko_attn_res against the reference's fixture
attnres.json (tests/golden/ref_attnres.npz) at its op tolerance and bitwise against the
compiled reference's k3_attn_res; one source returns that source; ko_moe_half with no
block residual is one step of ko_stack_step (h += MoE(RMSNorm(h))); ko_moe_half_v with a
block count per row (k3_ops.c:2481-2493) bitwise against the reference's own
k3_attn_res / k3_rmsnorm / k3_moe_prefill composed as the layer's MLP half
(refdrv_moe_half_v), and with one shared count equal to ko_moe_half."""
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


def half_v_inputs(L, T, maxb, seed):
    rng = np.random.default_rng(seed)
    H = L.H
    blocks = (rng.standard_normal((T, maxb, H)) * rng.uniform(0.2, 3, (T, maxb, 1))).astype(np.float32)
    pref = L.x(T, bf16=False, stream_sub=seed)
    fold = (rng.standard_normal(H) * 0.05).astype(np.float32)
    post = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    return blocks, pref, fold, post


def oracle_half_v(L, pref, blocks, nbv, nbs, fold, post, eps=1e-5):
    import ctypes as C
    from oracle_lib import I32P
    cfg = L.ko_cfg()
    w, cb, keep = L._weights()
    T = pref.shape[0]
    h = np.zeros_like(pref); p = pref.copy()
    nbv = np.ascontiguousarray(nbv, np.int32)
    d = oracle().ko_moe_half_v(ptr(h, F32P), ptr(p, F32P), ptr(blocks, F32P), blocks.shape[1],
                               ptr(nbv, I32P), nbs, ptr(fold, F32P), ptr(post, F32P), eps, T,
                               C.byref(cfg), C.byref(w))
    assert d == 0
    return h, p


def ref_half_v(ref_lib, L, pref, blocks, nbv, nbs, fold, post, eps=1e-5):
    import ctypes as C
    from oracle_lib import DrvCfg, I32P, KoExpert, U8P, vptr
    bank = (KoExpert * L.E)()
    keep = []
    for e in range(L.E):
        d = L.expert(e)
        keep.append(d)
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            setattr(bank[e], k, d[k].ctypes.data_as(U8P))
    dc = DrvCfg(L.H, L.latent, L.E, L.K, L.I, L.n_shared, L.renorm, L.latent_norm,
                L.routed_scale, L.rms_eps, L.situ_b1, L.situ_b2)
    T = pref.shape[0]
    h = np.zeros_like(pref); p = pref.copy()
    nbv = np.ascontiguousarray(nbv, np.int32)
    d = ref_lib.refdrv_moe_half_v(ptr(h, F32P), ptr(p, F32P), ptr(blocks, F32P),
                                  blocks.shape[1], ptr(nbv, I32P), nbs, ptr(fold, F32P),
                                  ptr(post, F32P), eps, T, C.byref(dc), ptr(L.gate, F32P),
                                  ptr(L.bias, F32P), bank, vptr(L.down), vptr(L.up),
                                  ptr(L.lnorm, F32P), vptr(L.sh1), vptr(L.sh3), vptr(L.sh2))
    assert d == 0
    return h, p


@pytest.mark.parametrize("latent", [False, True])
def test_moe_half_v_bitwise_vs_reference(ref_lib, latent):
    """Per-row counts 0 .. 4 in one call of 7 rows, and one shared count: the oracle's
    MLP half equals the reference's own functions composed as k3_decoder_layer_core does,
    bit for bit (h and pref)."""
    L = synth.tiny_latent(seed=41) if latent else synth.tiny(seed=41)
    T, maxb = 7, 5
    blocks, pref, fold, post = half_v_inputs(L, T, maxb, 3)
    for nbv, nbs in (([0, 3, 1, 4, 2, 0, 5], 1), ([2], 0)):
        h, p = oracle_half_v(L, pref, blocks, nbv, nbs, fold, post)
        rh, rp = ref_half_v(ref_lib, L, pref, blocks, nbv, nbs, fold, post)
        assert np.array_equal(h.view(np.uint32), rh.view(np.uint32))
        assert np.array_equal(p.view(np.uint32), rp.view(np.uint32))


def test_moe_half_v_rows_follow_their_counts():
    """Row t of a per-row call equals the single-row call with count nbv[t] (the counts
    reach their own rows, not their neighbours'), and a shared count equals ko_moe_half."""
    import ctypes as C
    L = synth.tiny(seed=42)
    T, maxb = 5, 4
    blocks, pref, fold, post = half_v_inputs(L, T, maxb, 9)
    nbv = [4, 0, 2, 1, 3]
    h, p = oracle_half_v(L, pref, blocks, nbv, 1, fold, post)
    for t in range(T):
        ht, pt = oracle_half_v(L, pref[t:t + 1].copy(), np.ascontiguousarray(blocks[t:t + 1]),
                               [nbv[t]], 0, fold, post)
        assert np.array_equal(h[t].view(np.uint32), ht[0].view(np.uint32))
    cfg = L.ko_cfg()
    w, cb, keep = L._weights()
    hs = np.zeros_like(pref); ps = pref.copy()
    oracle().ko_moe_half(ptr(hs, F32P), ptr(ps, F32P), ptr(blocks, F32P), maxb, 2,
                         ptr(fold, F32P), ptr(post, F32P), 1e-5, T, C.byref(cfg), C.byref(w))
    hv, pv = oracle_half_v(L, pref, blocks, [2], 0, fold, post)
    assert np.array_equal(hs.view(np.uint32), hv.view(np.uint32))
    # a mutation the test must catch: counts shifted by one row give other bits
    hx, _ = oracle_half_v(L, pref, blocks, nbv[1:] + nbv[:1], 1, fold, post)
    assert not np.array_equal(h.view(np.uint32), hx.view(np.uint32))
