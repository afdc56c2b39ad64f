"""Helpers shared by the GPU tests: device forward through the C ABI, layer builders."""
import sys

import numpy as np


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev_forward(torch, k3x, layer, x, bf16=False, resid=None):
    """Run k3x_moe_forward on device copies; returns (out, idx, wt) on the host."""
    T, H = x.shape
    K = layer.cfg.topk
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    if bf16:
        xt = xt.to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    idx = torch.full((T, K), -7, dtype=torch.int32, device="cuda")
    wt = torch.empty((T, K), dtype=torch.float32, device="cuda")
    rp = 0
    if resid is not None:
        rt = torch.from_numpy(np.ascontiguousarray(resid)).cuda()
        rp = rt.data_ptr()
    s = torch.cuda.current_stream()
    layer.forward(out.data_ptr(), xt.data_ptr(), T, k3x.K3X_BF16 if bf16 else k3x.K3X_F32,
                  rp, idx.data_ptr(), wt.data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    layer.check()
    return out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()


def layer_cfg(k3x, L):
    """k3x_cfg of a synth.Layer (betas of 2^64 are passed as they are: SwiGLU)."""
    return k3x.make_cfg(L.H, L.E, L.K, L.I, L.n_shared, L.renorm, L.routed_scale,
                        latent=L.latent, latent_norm=L.latent_norm, rms_eps=L.rms_eps,
                        situ_b1=L.situ_b1, situ_b2=L.situ_b2)


def bank_layer(k3x, L):
    return k3x.MoELayer.from_bank(layer_cfg(k3x, L), L.gate, L.bias, L.all_experts(), L.sh1,
                                  L.sh3, L.sh2, down=L.down, up=L.up, latent_norm=L.lnorm)


def synth_layer(k3x, L):
    return k3x.MoELayer.synthetic(layer_cfg(k3x, L), seed=L.seed, layer=L.layer,
                                  router_sigma=L.router_sigma, bias_sigma=L.bias_sigma,
                                  zipf_alpha=L.zipf_alpha, zipf_s=L.zipf_s,
                                  scale_lo=L.scale_lo, scale_hi=L.scale_hi,
                                  shared_sigma=L.shared_sigma, trunk_sigma=L.trunk_sigma)


def per_token_rel(out, ref):
    """Relative L2 distance of every row of out from the same row of ref."""
    d = np.linalg.norm((out - ref).astype(np.float64), axis=1)
    return d / np.maximum(np.linalg.norm(ref.astype(np.float64), axis=1), 1e-30)


def host_layer(L, x, experts):
    """The whole layer on the host for the rows of x, as the reference's prefill computes
    it (each row's result does not depend on the other rows of the call): the compiled
    reference where oracle/_ref is built -- refdrv_k2_prefill in the K2 form, the
    reference's k3_moe_prefill through refdrv_moe_cfg in the latent form, both equal to
    the oracle bit for bit on the CPU -- else the oracle's ko_moe_prefill.  `experts`, the
    rows' selections, are generated once and held for the call.  Returns (out, what ran)."""
    import ctypes as C
    import oracle_lib as ol

    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    L.hold(np.unique(experts))
    try:
        lib = ol.ref()
        if lib is None:
            return L.oracle_moe(x, prefill=True)[0], "the oracle's ko_moe_prefill"
        bank = (ol.KoExpert * L.E)()
        for e, d in L._held.items():
            for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
                setattr(bank[e], k, d[k].ctypes.data_as(ol.U8P))
        out = np.empty_like(x)
        if L.latent == 0:
            idx = np.empty((T, L.K), np.int32)
            wt = np.empty((T, L.K), np.float32)
            rc = lib.refdrv_k2_prefill(ol.ptr(out, ol.F32P), ol.ptr(x, ol.F32P), T, L.H, L.E,
                                       L.K, L.I, L.I * L.n_shared, L.routed_scale, L.renorm,
                                       ol.ptr(L.gate, ol.F32P), ol.ptr(L.bias, ol.F32P), bank,
                                       ol.ptr(L.sh1, ol.U16P), ol.ptr(L.sh3, ol.U16P),
                                       ol.ptr(L.sh2, ol.U16P), ol.ptr(idx, ol.I32P),
                                       ol.ptr(wt, ol.F32P))
            assert rc == 0
            return out, "the compiled reference's prefill (refdrv_k2_prefill)"
        dc = ol.DrvCfg(L.H, L.latent, L.E, L.K, L.I, L.n_shared, L.renorm, L.latent_norm,
                       L.routed_scale, L.rms_eps, L.situ_b1, L.situ_b2)
        idx = np.empty(L.K, np.int32)
        wt = np.empty(L.K, np.float32)
        gets = C.c_long(0)
        drops = lib.refdrv_moe_cfg(ol.ptr(out, ol.F32P), ol.ptr(x, ol.F32P), T, C.byref(dc),
                                   ol.ptr(L.gate, ol.F32P), ol.ptr(L.bias, ol.F32P), bank, None,
                                   ol.vptr(L.down), ol.vptr(L.up), ol.ptr(L.lnorm, ol.F32P),
                                   ol.vptr(L.sh1), ol.vptr(L.sh3), ol.vptr(L.sh2), 0, 1,
                                   ol.ptr(idx, ol.I32P), ol.ptr(wt, ol.F32P), C.byref(gets))
        assert drops == 0
        return out, "the compiled reference's k3_moe_prefill"
    finally:
        L.release()
