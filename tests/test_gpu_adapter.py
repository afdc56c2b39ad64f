"""The reference-side binding (kimi-k3-for-me_amd/csrc/k3x_ref_adapter.c) executed.

oracle/_ref/libk3adapter.so holds the binding compiled against the reference's own k3.h,
the reference's k3_ops.c (its k3_moe / k3_moe_prefill and k3_expert_drops) and the
harness oracle/ref_driver.c, which builds the reference's K3Cfg / K3MoeW / K3ExpertSrc
and calls one entry point (refdrv_moe_entry).  So the same layer goes through
k3_moe_gpu / k3_moe_prefill_gpu (libk3x on the device) and through the reference's CPU
k3_moe / k3_moe_prefill, in one process, with the caller's own types: the call site
k3_decoder_layer_core would use (k3_ops.c:2562-2567).

Branches: the K2-class emulation (identity latent, 2^64 betas: uploaded without
projections) and a LatentMoE layer, decode and prefill, against the reference and the
committed golden vectors; a cache-only draft over the source's resident() against the
reference's draft path; fp32 trunk weights refused (-1, the caller keeps its CPU path);
an expert that fails to load at upload counted in k3_expert_drops; the scratch query.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle_lib as ol
import refcall
import synth
from gpu_util import say

pytestmark = pytest.mark.gpu

TOL = 1e-3
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ADAPTER_SO = os.path.join(ol.ROOT, "oracle", "_ref", "libk3adapter.so")


@pytest.fixture(scope="module")
def adl(torch, k3x):
    if not os.path.exists(ADAPTER_SO):
        pytest.skip("oracle/_ref/libk3adapter.so not built (needs the reference tree)")
    lib = refcall.bind(C.CDLL(ADAPTER_SO))
    lib.refdrv_gpu_release.restype = None
    lib.k3_moe_gpu_scratch.restype = C.c_size_t
    lib.k3_moe_gpu_scratch.argtypes = [C.c_void_p, C.c_int]
    yield lib
    lib.refdrv_gpu_release()


Call = refcall.Call


@pytest.mark.parametrize("T,mode", [(1, 2), (8, 2), (8, 3), (40, 3)])
def test_k2_emulation_through_binding(adl, T, mode):
    """The K2-class layer as the reference expresses it (identity latent) through
    k3_moe_gpu (mode 2) or k3_moe_prefill_gpu (mode 3) against the reference's k3_moe /
    k3_moe_prefill on the same K3MoeW: the last token's routing exact, outputs within
    the parity bar; tokens 0..7 also against the committed golden vectors."""
    say(f"case: binding, K2 emulation, T={T}, {'k3_moe_prefill_gpu' if mode == 3 else 'k3_moe_gpu'}")
    adl.refdrv_gpu_release()
    L = synth.tiny(seed=0)
    c = Call(L, k2_emulation=True)
    x = L.x(T, bf16=False)
    go, gi, gw, gd, gs = c(adl, x, mode)
    ro, ri, rw, rd, rs = c(adl, x, mode - 2)
    assert gs == 0 and rs == 0 and gd == 0 and rd == 0
    # idx/wt: the last token's routing, except after a batched prefill of several tokens,
    # which leaves them untouched in both (k3_ops.c:2018-2053)
    assert np.array_equal(gi, ri)
    np.testing.assert_allclose(gw, rw, rtol=1e-6)
    if mode == 3 and T > 1:
        assert np.all(gi == -9) and np.all(gw == 0)
    err = synth.rel_l2(go, ro)
    say(f"  rel_l2 vs the reference's CPU path = {err:.3e}")
    assert err < TOL
    g = np.load(os.path.join(GOLD, "k2_tiny.npz"))
    n = min(T, 8)
    assert synth.rel_l2(go[:n], g["out"][:n]) < TOL
    if T <= 8 and not (mode == 3 and T > 1):
        assert np.array_equal(gi, g["idx"][T - 1])


@pytest.mark.parametrize("T,mode", [(6, 2), (6, 3), (20, 3)])
def test_latent_layer_through_binding(adl, T, mode):
    """A LatentMoE layer (latent 128, SiTU 4/25, latent RMSNorm, 2 shared experts) through
    the binding against the reference's CPU path and the k3_tiny golden vectors."""
    say(f"case: binding, LatentMoE layer, T={T}, mode {mode}")
    adl.refdrv_gpu_release()
    L = synth.tiny_latent(seed=0)
    c = Call(L, k2_emulation=False)
    x = L.x(T, bf16=False)
    go, gi, gw, gd, gs = c(adl, x, mode)
    ro, ri, rw, rd, rs = c(adl, x, mode - 2)
    assert gs == 0 and rs == 0 and gd == 0 and rd == 0
    assert np.array_equal(gi, ri) and np.array_equal(gw, rw)
    err = synth.rel_l2(go, ro)
    say(f"  rel_l2 vs the reference's CPU path = {err:.3e}")
    assert err < TOL
    g = np.load(os.path.join(GOLD, "k3_tiny.npz"))
    n = min(T, 6)
    assert synth.rel_l2(go[:n], g["out"][:n]) < TOL


@pytest.mark.parametrize("T,mode", [(1, 2), (5, 2), (20, 3)])
def test_cache_only_draft_through_binding(adl, T, mode):
    """A cache-only draft (K3MoeW.cache_only with the source's resident() reporting a
    mask) through the binding, against the reference's CPU path with the same source:
    the last token's indices exact and weights to float rounding, outputs within the
    parity bar."""
    say(f"case: binding, cache-only draft over a half-resident source, T={T}, mode {mode}")
    adl.refdrv_gpu_release()
    L = synth.tiny(seed=9)
    c = Call(L, k2_emulation=True)
    res = (np.random.default_rng(T).random(L.E) < 0.5).astype(np.int32)
    x = L.x(T, bf16=False)
    go, gi, gw, gd, gs = c(adl, x, mode, cache_only=1, res=res)
    ro, ri, rw, rd, rs = c(adl, x, mode - 2, cache_only=1, res=res)
    assert gs == 0 and rs == 0 and gd == 0 and rd == 0
    assert np.array_equal(gi, ri)
    np.testing.assert_allclose(gw, rw, rtol=1e-6)
    err = synth.rel_l2(go, ro)
    say(f"  rel_l2 vs the reference's CPU path = {err:.3e}")
    assert err < TOL
    o, oi, _ = L.oracle_moe_cache_only(x, res)
    assert np.array_equal(gi, oi[-1]) and synth.rel_l2(go, o) < TOL


def test_binding_refusals_and_drops(adl, k3x):
    """What the binding does not run returns -1 with the output untouched (the caller
    keeps its CPU path): fp32 trunk weights.  An expert whose fetch fails at upload
    counts once in k3_expert_drops (and in k3x_expert_drops), the call returns -1; the
    next call with a working source uploads and runs."""
    say("case: binding refusal (fp32 trunk) and an upload drop")
    adl.refdrv_gpu_release()
    L = synth.tiny(seed=3)
    c = Call(L, k2_emulation=True)
    x = L.x(2, bf16=False)
    for kw in ({"trunk_f32": 1},):
        o, i, w, d, s = c(adl, x, 2, **kw)
        assert s == -1 and d == 0, kw
        assert np.all(o == np.float32(7.0)) and np.all(i == -9), kw
    fail = np.zeros(L.E, np.int32)
    fail[5] = 1
    d0 = k3x.expert_drops()
    o, i, w, d, s = c(adl, x, 2, fail=fail)
    assert s == -1 and d == 1
    assert k3x.expert_drops() == d0 + 1
    o, i, w, d, s = c(adl, x, 2)
    ro, ri, _, _, _ = c(adl, x, 0)
    assert s == 0 and d == 0 and np.array_equal(i, ri)
    assert synth.rel_l2(o, ro) < TOL
    assert adl.k3_moe_gpu_scratch(None, 8) == 0


@pytest.mark.parametrize("slots,T,mode", [("6", 1, 2), ("12", 3, 2), ("16", 20, 3)])
def test_binding_over_an_expert_cache(adl, slots, T, mode, monkeypatch):
    """K3X_ADAPTER_SLOTS makes the binding keep the layer as an HBM expert cache fed by
    the reference's own source (what it does when a whole layer does not fit): against
    the reference's CPU path with the same source.  A call whose tokens name more experts
    than the slots returns -1 (the caller's CPU path runs it)."""
    say(f"case: binding over an expert cache of {slots} slots, T={T}, mode {mode}")
    monkeypatch.setenv("K3X_ADAPTER_SLOTS", slots)
    adl.refdrv_gpu_release()
    L = synth.tiny(seed=10)
    c = Call(L, k2_emulation=True)
    x = L.x(T, bf16=False)
    go, gi, gw, gd, gs = c(adl, x, mode)
    ro, ri, rw, rd, rs = c(adl, x, mode - 2)
    assert gs == 0 and rs == 0 and gd == 0 and rd == 0
    assert np.array_equal(gi, ri)
    err = synth.rel_l2(go, ro)
    say(f"  rel_l2 vs the reference's CPU path = {err:.3e}")
    assert err < TOL
    if slots == "6":
        x3 = L.x(3, bf16=False)
        _, i3, _, _ = L.oracle_moe(x3)
        assert len(np.unique(i3)) > 6
        o, i, w, d, s = c(adl, x3, 2)
        assert s == -1 and d == 0 and np.all(o == np.float32(7.0))
    adl.refdrv_gpu_release()
