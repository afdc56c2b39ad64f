"""Writes the committed golden fixtures under tests/golden/ (run in a container that has
the reference tree; the GPU side only reads the .npz files).

1. The reference's own op fixtures for this path, converted from JSON to compact .npz
   (data only): tests/fixtures/ops/{router,situ_glu,rmsnorm}.json and
   tests/fixtures/mxfp4.json (real checkpoint MXFP4 bytes with their exact dequant).
   tests/fixtures/ops/moe.json (the whole LatentMoE block, fp32 experts and trunk) goes
   to ref_moe_latent.npz, tests/fixtures/ops/attnres.json to ref_attnres.npz.
2. Whole-layer golden vectors of the K2-class layer computed by the COMPILED REFERENCE
   (oracle/_ref/libk3ref.so: the reference's k3_ops.c, k3_moe/k3_moe_prefill with
   identity latent projections and 2^64 SiTU betas) on seeded synthetic layers:
     k2_tiny.npz  hidden 256, 16 experts top-4, I 128, 1 shared; 8 fp32 tokens; every
                  output, index and weight (weights regenerate from the seed).
     k2_full.npz  hidden 7168, 384 experts top-8, I 2048, 1 shared; 2 bf16 tokens
                  (normal bias) and 2 with Zipf bias; indices, weights, every 16th output
                  row element and an FNV-1a hash of the full output bits.
   and of the K3 LatentMoE layer, the reference's k3_moe with real down/up projections:
     k3_tiny.npz  hidden 256, latent 128, 16 experts top-4, I 128, 2 shared, SiTU 4/25,
                  latent RMSNorm; 6 fp32 tokens; every output, index and weight.

Usage: make -C oracle && make -C oracle ref && python tests/golden/make_golden.py
"""
import ctypes as C
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as ol  # noqa: E402
import synth  # noqa: E402

FIX = "/root/reference/tests/fixtures"


def arr(d):
    return np.asarray(d["data"], dtype=np.float64)


def convert_ops():
    r = json.load(open(os.path.join(FIX, "ops", "router.json")))
    np.savez_compressed(os.path.join(HERE, "ref_router.npz"),
                        gate=arr(r["gate_weight"]).astype(np.float32).reshape(r["gate_weight"]["shape"]),
                        bias=arr(r["bias"]).astype(np.float32),
                        x=arr(r["in"]).astype(np.float32).reshape(r["in"]["shape"]),
                        topk_idx=arr(r["topk_idx"]).astype(np.int32).reshape(r["topk_idx"]["shape"]),
                        topk_weight=arr(r["topk_weight"]).astype(np.float32).reshape(r["topk_weight"]["shape"]),
                        top_k=r["top_k"], n_experts=r["n_experts"],
                        rows_bias_changed=r["rows_where_bias_changed_selection"])
    s = json.load(open(os.path.join(FIX, "ops", "situ_glu.json")))
    np.savez_compressed(os.path.join(HERE, "ref_situ_glu.npz"),
                        x=arr(s["in"]).astype(np.float32).reshape(s["in"]["shape"]),
                        out=arr(s["out"]).astype(np.float32).reshape(s["out"]["shape"]),
                        beta=s["beta"], linear_beta=s["linear_beta"])
    m = json.load(open(os.path.join(FIX, "ops", "rmsnorm.json")))
    np.savez_compressed(os.path.join(HERE, "ref_rmsnorm.npz"),
                        w=arr(m["weight"]).astype(np.float32),
                        x=arr(m["in"]).astype(np.float32).reshape(m["in"]["shape"]),
                        out=arr(m["out"]).astype(np.float32).reshape(m["out"]["shape"]),
                        eps=m["eps"])
    man = json.load(open(os.path.join(FIX, "ops", "MANIFEST.json")))
    q = json.load(open(os.path.join(FIX, "mxfp4.json")))
    np.savez_compressed(os.path.join(HERE, "ref_mxfp4.npz"),
                        packed=np.asarray(q["packed"]["data"], np.uint8).reshape(q["packed"]["shape"]),
                        scales=np.asarray(q["scales"]["data"], np.uint8).reshape(q["scales"]["shape"]),
                        expected=np.asarray(q["expected"]["data"], np.float32).reshape(q["expected"]["shape"]),
                        swapped_first64=np.asarray(q["expected_swapped_nibbles"]["first64"], np.float32),
                        lut=np.asarray(q["e2m1_lut"], np.float32), group=q["group_size"],
                        tol_abs=man["tolerance"]["fp32_abs"], tol_rel=man["tolerance"]["fp32_rel"])
    mo = json.load(open(os.path.join(FIX, "ops", "moe.json")))
    rec = {k: mo[k] for k in ("hidden", "latent", "moe_inter", "n_experts", "top_k", "n_shared",
                              "routed_scale", "renorm", "latent_norm", "rms_eps", "situ_b1",
                              "situ_b2")}
    for k, v in mo.items():
        if isinstance(v, dict) and "data" in v:
            rec[k] = arr(v).astype(np.float32).reshape(v["shape"])
    rec["tol_abs"] = man["tolerance"]["fp32_abs"]
    rec["tol_rel"] = man["tolerance"]["fp32_rel"]
    np.savez_compressed(os.path.join(HERE, "ref_moe_latent.npz"), **rec)
    a = json.load(open(os.path.join(FIX, "ops", "attnres.json")))
    np.savez_compressed(os.path.join(HERE, "ref_attnres.npz"),
                        prefix=arr(a["prefix_sum"]).astype(np.float32).reshape(a["prefix_sum"]["shape"]),
                        blocks=arr(a["block_residual"]).astype(np.float32).reshape(a["block_residual"]["shape"]),
                        fold=arr(a["fold_hint"]).astype(np.float32),
                        out=arr(a["out"]).astype(np.float32).reshape(a["out"]["shape"]),
                        eps=a["eps"], n_sources=a["n_sources"],
                        tol_abs=man["tolerance"]["fp32_abs"], tol_rel=man["tolerance"]["fp32_rel"])


def ref_moe(L, x, prefill=False):
    ref = ol.ref()
    T = x.shape[0]
    bank = (ol.KoExpert * L.E)()
    keep = []
    for e in range(L.E):
        d = L.expert(e)
        keep.append(d)
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            setattr(bank[e], k, d[k].ctypes.data_as(ol.U8P))
    out = np.empty_like(x)
    idx = np.empty(L.K, np.int32)
    wt = np.empty(L.K, np.float32)
    gets = C.c_long(0)
    drops = ref.refdrv_moe(ol.ptr(out, ol.F32P), ol.ptr(x, ol.F32P), T, L.H, L.E, L.K, L.I,
                           L.n_shared, L.routed_scale, L.renorm, ol.ptr(L.gate, ol.F32P),
                           ol.ptr(L.bias, ol.F32P), bank, None, ol.ptr(L.sh1, ol.U16P),
                           ol.ptr(L.sh3, ol.U16P), ol.ptr(L.sh2, ol.U16P), 1 if prefill else 0,
                           ol.ptr(idx, ol.I32P), ol.ptr(wt, ol.F32P), C.byref(gets))
    assert drops == 0
    return out, idx, wt


def ref_moe_cfg(L, x, prefill=False):
    """k3_moe / k3_moe_prefill of the compiled reference on a layer in general form."""
    ref = ol.ref()
    T = x.shape[0]
    bank = (ol.KoExpert * L.E)()
    keep = []
    for e in range(L.E):
        d = L.expert(e)
        keep.append(d)
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            setattr(bank[e], k, d[k].ctypes.data_as(ol.U8P))
    dc = ol.DrvCfg(L.H, L.latent, L.E, L.K, L.I, L.n_shared, L.renorm, L.latent_norm,
                   L.routed_scale, L.rms_eps, L.situ_b1, L.situ_b2)
    out = np.empty_like(x)
    idx = np.empty(L.K, np.int32)
    wt = np.empty(L.K, np.float32)
    gets = C.c_long(0)
    drops = ref.refdrv_moe_cfg(ol.ptr(out, ol.F32P), ol.ptr(x, ol.F32P), T, C.byref(dc),
                               ol.ptr(L.gate, ol.F32P), ol.ptr(L.bias, ol.F32P), bank, None,
                               ol.vptr(L.down), ol.vptr(L.up), ol.ptr(L.lnorm, ol.F32P),
                               ol.vptr(L.sh1), ol.vptr(L.sh3), ol.vptr(L.sh2), 0,
                               1 if prefill else 0, ol.ptr(idx, ol.I32P), ol.ptr(wt, ol.F32P),
                               C.byref(gets))
    assert drops == 0
    return out, idx, wt, gets.value


def fnv1a(a):
    h = 0xCBF29CE484222325
    for b in np.ascontiguousarray(a).view(np.uint8).tobytes():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def route_ref(L, x):
    """Every token's routing through the compiled reference's k3_router."""
    ref = ol.ref()
    T = x.shape[0]
    idx = np.empty((T, L.K), np.int32)
    wt = np.empty((T, L.K), np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        ref.k3_router(ol.ptr(idx[t], ol.I32P), ol.ptr(wt[t], ol.F32P), ol.ptr(xt, ol.F32P),
                      ol.ptr(L.gate, ol.F32P), ol.ptr(L.bias, ol.F32P), L.H, L.E, L.K,
                      L.renorm, L.routed_scale)
    return idx, wt


def k2_tiny():
    L = synth.tiny(seed=0)
    x = L.x(8, bf16=False)
    outs = np.stack([ref_moe(L, x[t:t + 1])[0][0] for t in range(8)])
    idx, wt = route_ref(L, x)
    np.savez_compressed(os.path.join(HERE, "k2_tiny.npz"), out=outs, idx=idx, wt=wt, seed=0,
                        T=8)


def k3_tiny():
    """The small LatentMoE layer (synth.tiny_latent, seed 0): 6 fp32 tokens through the
    reference's k3_moe in one call; every output, index and weight."""
    L = synth.tiny_latent(seed=0)
    x = L.x(6, bf16=False)
    out = ref_moe_cfg(L, x)[0]
    idx, wt = route_ref(L, x)
    np.savez_compressed(os.path.join(HERE, "k3_tiny.npz"), out=out, idx=idx, wt=wt, seed=0,
                        T=6)


def k2_full():
    rec = {}
    for name, kw, sub in (("normal", {}, 0), ("zipf", {"zipf_alpha": 1.0}, 1)):
        L = synth.full(seed=1, **kw)
        x = L.x(2, bf16=True, stream_sub=sub)
        idx, wt = route_ref(L, x)
        full_out = ref_moe(L, np.ascontiguousarray(x))[0]
        outs, hashes = [], []
        for t in range(2):
            o = full_out[t]
            outs.append(o[::16].copy())
            hashes.append(fnv1a(o))
        rec[name + "_idx"] = idx
        rec[name + "_wt"] = wt
        rec[name + "_out16"] = np.stack(outs)
        rec[name + "_hash"] = np.array(hashes, np.uint64)
    np.savez_compressed(os.path.join(HERE, "k2_full.npz"), **rec)


if __name__ == "__main__":
    ol.oracle()
    assert ol.ref() is not None, "build oracle/_ref first (make -C oracle ref)"
    convert_ops()
    k2_tiny()
    k3_tiny()
    if "--no-full" not in sys.argv:
        k2_full()
    print("golden fixtures written to", HERE)
