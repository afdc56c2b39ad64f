"""The oracle's cache-only (draft) routing, ko_moe_cache_only, bitwise against the
compiled reference's k3_moe / k3_moe_prefill with K3MoeW.cache_only set and a
resident() that reports a given mask (oracle/ref_driver.c, k3_ops.c:1884-1926, :2018):
outputs, the last token's idx/wt (kept experts first, the router's values after them),
over an all-resident mask (the exact routing with its weights renormalised to sum 1), an
empty one (shared expert only) and random ones, for a K2-class layer and a LatentMoE
layer."""
import numpy as np
import pytest

import oracle_lib as ol
import refcall
import synth


@pytest.fixture(scope="module")
def rlib():
    lib = ol.ref()
    if lib is None:
        pytest.skip("compiled reference (oracle/_ref) not built: reference tree absent")
    return refcall.bind(lib)


@pytest.mark.parametrize("kind", ["k2", "latent"])
@pytest.mark.parametrize("mask", ["all", "none", "half", "sparse"])
@pytest.mark.parametrize("mode", [0, 1])
def test_cache_only_bitwise_vs_reference(rlib, kind, mask, mode):
    L = synth.tiny(seed=21) if kind == "k2" else synth.tiny_latent(seed=2)
    rng = np.random.default_rng(5)
    res = {"all": np.ones(L.E, np.int32), "none": np.zeros(L.E, np.int32),
           "half": (rng.random(L.E) < 0.5).astype(np.int32),
           "sparse": (rng.random(L.E) < 0.15).astype(np.int32)}[mask]
    c = refcall.Call(L, k2_emulation=(kind == "k2"))
    x = L.x(5, bf16=False)
    o, idx, wt = L.oracle_moe_cache_only(x, res)
    r, ri, rw, rd, st = c(rlib, x, mode, cache_only=1, res=res)
    assert st == 0 and rd == 0
    assert np.array_equal(o.view(np.uint32), r.view(np.uint32))
    assert np.array_equal(idx[-1], ri) and np.array_equal(wt[-1].view(np.uint32), rw.view(np.uint32))
    if mask == "all":
        # every expert kept: the exact routing, its weights divided by their sum (so the
        # routed scale is divided out too: the draft's mixture sums to 1)
        _, ei, ew, _ = L.oracle_moe(x)
        assert np.array_equal(idx, ei)
        for t in range(x.shape[0]):
            s = np.float32(0)
            for j in range(L.K):
                s = np.float32(s + ew[t, j])
            assert np.array_equal(wt[t], (ew[t] / s).astype(np.float32))


def test_cache_only_semantics():
    """Kept experts first in top-k order, their weights summing to 1 (the routed scale
    is divided out with the rest), the router's entries after them; a layer without
    resident experts gives the shared expert alone."""
    L = synth.tiny(seed=22)
    res = np.zeros(L.E, np.int32)
    res[::3] = 1
    x = L.x(4, bf16=False)
    _, ei, ew, _ = L.oracle_moe(x)
    o, idx, wt = L.oracle_moe_cache_only(x, res)
    for t in range(4):
        kept = [j for j in range(L.K) if res[ei[t, j]]]
        m = len(kept)
        assert list(idx[t, :m]) == [ei[t, j] for j in kept]
        assert list(idx[t, m:]) == list(ei[t, m:])
        if m:
            assert abs(float(np.sum(wt[t, :m], dtype=np.float64)) - 1.0) < 1e-6
    L0 = synth.tiny(seed=22, n_shared=0)
    o0, _, _ = L0.oracle_moe_cache_only(x, np.zeros(L.E, np.int32))
    assert np.all(o0 == 0)
