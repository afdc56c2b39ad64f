"""Pins the oracle's K3 LatentMoE form (ko_moe / ko_moe_prefill with cfg.latent > 0)
against:
  * the reference's own whole-block fixture tests/fixtures/ops/moe.json (fp32 experts and
    trunk, SiTU driven into its caps, a bias that reorders the top-k; converted to
    tests/golden/ref_moe_latent.npz), at the reference's op tolerance (MANIFEST.json);
  * the compiled reference's k3_moe and k3_moe_prefill (oracle/_ref), bit for bit, on
    seeded MXFP4 layers with bf16 trunk matrices, and golden vectors it wrote
    (tests/golden/k3_tiny.npz);
  * what the mathematics fixes: with latent = hidden, identity down/up, no latent norm and
    2^64 betas the form is the K2-class layer bit for bit; with the latent norm on, the
    output does not change when every routing weight is doubled (the norm is on the
    aggregate: a norm per expert, or none, scales with the weights).
"""
import ctypes as C
import os

import numpy as np
import pytest

import synth
from oracle_lib import (F32P, GET_FN, I32P, KoCfg, KoExpert, KoWeights, U8P, oracle, ptr,
                        vptr)

HERE = os.path.dirname(os.path.abspath(__file__))


def gold(name):
    return np.load(os.path.join(HERE, "golden", name), allow_pickle=False)


@pytest.fixture(scope="module")
def ref_lib():
    from oracle_lib import ref
    r = ref()
    if r is None:
        pytest.skip("compiled reference not built (make -C oracle ref)")
    return r


def ref_moe_cfg(ref_lib, L, x, prefill, fail=None):
    from oracle_lib import DrvCfg
    bank = (KoExpert * L.E)()
    keep = []
    for e in range(L.E):
        d = L.expert(e)
        keep.append(d)
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            setattr(bank[e], k, d[k].ctypes.data_as(U8P))
    dc = DrvCfg(L.H, L.latent, L.E, L.K, L.I, L.n_shared, L.renorm, L.latent_norm,
                L.routed_scale, L.rms_eps, L.situ_b1, L.situ_b2)
    out = np.empty_like(x)
    idx = np.empty(L.K, np.int32)
    wt = np.empty(L.K, np.float32)
    gets = C.c_long(0)
    fa = None
    if fail is not None:
        fa = np.zeros(L.E, np.int32)
        fa[list(fail)] = 1
    drops = ref_lib.refdrv_moe_cfg(ptr(out, F32P), ptr(x, F32P), x.shape[0], C.byref(dc),
                                   ptr(L.gate, F32P), ptr(L.bias, F32P), bank,
                                   ptr(fa, I32P) if fa is not None else None, vptr(L.down),
                                   vptr(L.up), ptr(L.lnorm, F32P), vptr(L.sh1), vptr(L.sh3),
                                   vptr(L.sh2), 0, 1 if prefill else 0, ptr(idx, I32P),
                                   ptr(wt, F32P), C.byref(gets))
    return out, idx, wt, drops, gets.value


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ the reference's fixture
def test_latent_moe_reference_fixture():
    """moe.json through ko_moe: fp32 trunk (trunk_f32) and the resident fp32 expert bank
    (get == NULL), T = 3, compared at atol 1e-5 / rtol 1e-4 (test_ops.c:694-774)."""
    g = gold("ref_moe_latent.npz")
    H, LT, I = int(g["hidden"]), int(g["latent"]), int(g["moe_inter"])
    E, K, NS = int(g["n_experts"]), int(g["top_k"]), int(g["n_shared"])
    cfg = KoCfg(H, E, K, I, NS, int(g["renorm"]), float(g["routed_scale"]),
                float(g["situ_b1"]), float(g["situ_b2"]), 32, LT, int(g["latent_norm"]),
                float(g["rms_eps"]))
    f = lambda k: np.ascontiguousarray(g[k], np.float32)
    W1 = np.ascontiguousarray(np.stack([f(f"experts_{e}_w1_weight") for e in range(E)]))
    W3 = np.ascontiguousarray(np.stack([f(f"experts_{e}_w3_weight") for e in range(E)]))
    W2 = np.ascontiguousarray(np.stack([f(f"experts_{e}_w2_weight") for e in range(E)]))
    arrs = {k: f(k) for k in ("gate_weight", "e_score_correction_bias", "down_weight",
                              "up_weight", "norm_weight", "shared_w1_weight",
                              "shared_w3_weight", "shared_w2_weight")}
    w = KoWeights(ptr(arrs["gate_weight"], F32P), ptr(arrs["e_score_correction_bias"], F32P),
                  GET_FN(), None,        # a NULL get(): the resident fp32 bank
                  vptr(arrs["shared_w1_weight"]), vptr(arrs["shared_w3_weight"]),
                  vptr(arrs["shared_w2_weight"]), vptr(arrs["down_weight"]),
                  vptr(arrs["up_weight"]), ptr(arrs["norm_weight"], F32P), 1,
                  ptr(W1, F32P), ptr(W3, F32P), ptr(W2, F32P))
    x = f("in").reshape(-1, H)
    T = x.shape[0]
    out = np.empty_like(x)
    idx = np.empty((T, K), np.int32)
    wt = np.empty((T, K), np.float32)
    drops = oracle().ko_moe(ptr(out, F32P), ptr(x, F32P), T, C.byref(cfg), C.byref(w),
                            ptr(idx, I32P), ptr(wt, F32P))
    assert drops == 0
    want = f("out").reshape(-1, H)
    np.testing.assert_allclose(out, want, atol=float(g["tol_abs"]), rtol=float(g["tol_rel"]))
    # the fixture exercises what it says: SiTU saturates, the bias reorders the top-k
    b1 = float(g["situ_b1"])
    z = np.stack([arrs["down_weight"].astype(np.float64) @ x[t] for t in range(T)])
    gate = np.einsum("eil,tl->tei", W1.astype(np.float64), z)
    assert np.abs(gate).max() > 2 * b1
    logits = x.astype(np.float64) @ arrs["gate_weight"].astype(np.float64).T
    plain = np.argsort(-logits, axis=1, kind="stable")[:, :K]
    assert any(set(plain[t]) != set(idx[t]) for t in range(T))


# ------------------------------------------------------------ the compiled reference
@pytest.mark.parametrize("seed", [0, 2])
def test_latent_moe_bitwise_vs_reference(seed, ref_lib):
    L = synth.tiny_latent(seed=seed)
    x = L.x(6, bf16=False)
    o, idx, wt, d = L.oracle_moe(x)
    r, ri, rw, rd, _ = ref_moe_cfg(ref_lib, L, x, prefill=False)
    assert d == 0 and rd == 0
    assert np.array_equal(bits(o), bits(r))
    assert np.array_equal(idx[-1], ri) and np.array_equal(bits(wt[-1]), bits(rw))


def test_latent_moe_prefill_bitwise(ref_lib):
    """The reference's t_moe_prefill shape (test_ops.c:884-1014): hidden = latent = 64,
    I 64, top-16 of 40, one shared expert, routed_scale 2.5, latent norm, SiTU 4/25, T =
    130 over 64-token sub-chunks: ko_moe_prefill equals ko_moe and the reference's
    k3_moe_prefill bit for bit, with one get() per unique expert per sub-chunk."""
    L = synth.Layer(H=64, E=40, K=16, I=64, n_shared=1, latent=64, latent_norm=1,
                    situ_b1=4.0, situ_b2=25.0, routed_scale=2.5, seed=7, trunk_sigma=0.125,
                    scale_lo=121, scale_hi=124)
    x = L.x(130, bf16=False)
    op, pidx, pwt, pd, ng = L.oracle_moe(x, prefill=True)
    o, idx, wt, d = L.oracle_moe(x)
    assert pd == 0 and d == 0
    assert np.array_equal(bits(op), bits(o))
    assert np.array_equal(pidx, idx)
    want_gets = sum(len(np.unique(idx[t0:t0 + 64])) for t0 in range(0, 130, 64))
    assert ng == want_gets
    r, _, _, rd, rg = ref_moe_cfg(ref_lib, L, x, prefill=True)
    assert rd == 0 and rg == want_gets
    assert np.array_equal(bits(op), bits(r))


def test_latent_moe_drop_vs_reference(ref_lib):
    L = synth.tiny_latent(seed=1)
    x = L.x(3, bf16=False)
    o, idx, _, _ = L.oracle_moe(x)
    victim = int(idx[0, 1])
    od, _, _, drops = L.oracle_moe(x, fail={victim})
    assert drops == int((idx == victim).sum())
    r, _, _, rd, _ = ref_moe_cfg(ref_lib, L, x, prefill=False, fail={victim})
    assert rd == drops
    assert np.array_equal(bits(od), bits(r))


def test_golden_k3_tiny():
    g = gold("k3_tiny.npz")
    L = synth.tiny_latent(seed=int(g["seed"]))
    x = L.x(int(g["T"]), bf16=False)
    o, idx, wt, _ = L.oracle_moe(x)
    assert np.array_equal(idx, g["idx"])
    assert np.array_equal(bits(wt), bits(g["wt"]))
    assert np.array_equal(bits(o), bits(g["out"]))


# ------------------------------------------------------------ what the mathematics fixes
def test_identity_latent_is_the_k2_layer():
    """latent = hidden with bf16 identity down/up, no latent norm and 2^64 betas: the
    projections are exact, so the output is the K2-class form's (latent = 0) bit for bit."""
    K2 = synth.tiny(seed=5)
    x = K2.x(4, bf16=False)
    want, widx, wwt, _ = K2.oracle_moe(x)
    eye = np.zeros((K2.H, K2.H), np.uint16)
    eye[np.arange(K2.H), np.arange(K2.H)] = 0x3F80
    K2.latent, K2.down, K2.up = K2.H, eye, eye
    got, idx, wt, _ = K2.oracle_moe(x)
    assert np.array_equal(idx, widx)
    assert np.array_equal(bits(got), bits(want))


def test_latent_norm_is_on_the_aggregate():
    """Doubling routed_scale doubles every routed contribution exactly; RMSNorm of the
    aggregate cancels that up to eps, so the output barely moves.  Without the latent norm
    the routed part doubles, which this data shows too."""
    def run(scale, norm):
        L = synth.tiny_latent(seed=3, routed_scale=scale, n_shared=0, latent_norm=norm)
        if not norm:
            L.lnorm = None
        return L.oracle_moe(L.x(4, bf16=False))[0]
    a, b = run(1.0, 1), run(2.0, 1)
    assert synth.rel_l2(b, a) < 1e-5
    c, d = run(1.0, 0), run(2.0, 0)
    assert synth.rel_l2(d, 2 * c) < 1e-6 and synth.rel_l2(d, c) > 0.5
