"""Calls into oracle/ref_driver.c's refdrv_moe_entry: one MoE layer through the reference's
own K3MoeW / K3Cfg / K3ExpertSrc, on the reference's CPU path (modes 0 k3_moe, 1
k3_moe_prefill) or, in the adapter library, through the GPU binding (modes 2
k3_moe_gpu, 3 k3_moe_prefill_gpu)."""
import ctypes as C

import numpy as np

import oracle_lib as ol


def bind(lib):
    lib.refdrv_moe_entry.restype = C.c_long
    lib.refdrv_moe_entry.argtypes = [
        ol.F32P, ol.F32P, C.c_int, C.POINTER(ol.DrvCfg), ol.F32P, ol.F32P,
        C.POINTER(ol.KoExpert), ol.I32P, C.c_void_p, C.c_void_p, ol.F32P, C.c_void_p,
        C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, ol.I32P, ol.I32P, ol.F32P,
        C.POINTER(C.c_int), C.POINTER(C.c_long)]
    return lib


def identity_bf16(n):
    m = np.zeros((n, n), np.uint16)
    m[np.arange(n), np.arange(n)] = 0x3F80
    return m


class Call:
    """The layer's arrays in the reference's types, kept alive across calls."""

    def __init__(self, L, k2_emulation):
        self.L = L
        self.bank = (ol.KoExpert * L.E)()
        self.keep = []
        for e in range(L.E):
            d = L.expert(e)
            self.keep.append(d)
            for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
                setattr(self.bank[e], k, d[k].ctypes.data_as(ol.U8P))
        if k2_emulation:
            # K2 through the reference's own types: latent = hidden, identity down/up,
            # latent norm off, SiTU betas 2^64 (SwiGLU)
            self.down = self.up = identity_bf16(L.H)
            self.dc = ol.DrvCfg(L.H, L.H, L.E, L.K, L.I, L.n_shared, L.renorm, 0,
                                L.routed_scale, L.rms_eps, 2.0 ** 64, 2.0 ** 64)
        else:
            self.down, self.up = L.down, L.up
            self.dc = ol.DrvCfg(L.H, L.latent, L.E, L.K, L.I, L.n_shared, L.renorm,
                                L.latent_norm, L.routed_scale, L.rms_eps, L.situ_b1, L.situ_b2)

    def __call__(self, lib, x, mode, fail=None, cache_only=0, trunk_f32=0, res=None):
        """out, idx [K] (the last token's, as the reference leaves it), wt, drops, status."""
        L = self.L
        x = np.ascontiguousarray(x, np.float32)
        out = np.full_like(x, np.float32(7.0))
        idx = np.full(L.K, -9, np.int32)
        wt = np.zeros(L.K, np.float32)
        st = C.c_int(99)
        gets = C.c_long(0)
        fa = None if fail is None else np.ascontiguousarray(fail, np.int32)
        ra = None if res is None else np.ascontiguousarray(res, np.int32)
        drops = lib.refdrv_moe_entry(
            ol.ptr(out, ol.F32P), ol.ptr(x, ol.F32P), x.shape[0], C.byref(self.dc),
            ol.ptr(L.gate, ol.F32P), ol.ptr(L.bias, ol.F32P), self.bank, ol.ptr(fa, ol.I32P),
            ol.vptr(self.down), ol.vptr(self.up), ol.ptr(L.lnorm, ol.F32P), ol.vptr(L.sh1),
            ol.vptr(L.sh3), ol.vptr(L.sh2), trunk_f32, mode, cache_only, ol.ptr(ra, ol.I32P),
            ol.ptr(idx, ol.I32P), ol.ptr(wt, ol.F32P), C.byref(st), C.byref(gets))
        return out, idx, wt, drops, st.value
