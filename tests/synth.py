"""Seeded MoE layers on the host, from the oracle's counter-based generator.

Test infrastructure.  The product library has its own implementation of the same rule
(k3x_synth_*); tests/test_abi.py checks the two agree bit for bit, so a layer built here
and one built by k3x_synth_layer_create hold the same weights.

Streams follow include/k3x_moe.h: router 0, bias 1, x 2, sh1 3, sh3 4, sh2 5, norm 6,
latent down 7, latent up 8, latent norm 9, expert codes 10 and scales 11 with
sub = 3*expert + {0 gate, 1 up, 2 down}.

A layer with latent > 0 is the K3 LatentMoE form: experts at the latent width, bf16
down [latent][H] and up [H][latent], the latent RMSNorm weights when latent_norm, and
SiTU betas; latent == 0 is the K2-class form.
"""
import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from oracle_lib import (F32P, GET_FN, I32P, KoCfg, KoExpert, KoWeights, U8P, U16P, oracle,
                        ptr, vptr)

S_ROUTER, S_BIAS, S_X, S_SH1, S_SH3, S_SH2, S_NORM, S_DOWN, S_UP, S_LNORM = range(10)
S_CODES, S_SCALES = 10, 11


def key(seed, layer, stream, sub=0):
    return oracle().ko_key(seed, layer, stream, sub)


def normal_f32(n, k, mu=0.0, sigma=1.0):
    a = np.empty(n, np.float32)
    oracle().ko_fill_normal_f32(ptr(a, F32P), n, k, mu, sigma)
    return a


def normal_bf16(n, k, mu=0.0, sigma=1.0):
    a = np.empty(n, np.uint16)
    oracle().ko_fill_normal_bf16(ptr(a, U16P), n, k, mu, sigma)
    return a


def codes(n, k):
    a = np.empty(n, np.uint8)
    oracle().ko_fill_codes(ptr(a, U8P), n, k)
    return a


def scales(n, k, lo, hi):
    a = np.empty(n, np.uint8)
    oracle().ko_fill_scales(ptr(a, U8P), n, k, lo, hi)
    return a


def bf16_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


@dataclass
class Layer:
    H: int
    E: int
    K: int
    I: int
    n_shared: int = 1
    seed: int = 0
    layer: int = 0
    router_sigma: float = 0.02
    bias_sigma: float = 0.1
    zipf_alpha: float = 0.0
    zipf_s: float = 1.1
    scale_lo: int = 121
    scale_hi: int = 125
    shared_sigma: float = 0.02
    routed_scale: float = 2.5
    renorm: int = 1
    latent: int = 0
    latent_norm: int = 0
    situ_b1: float = 2.0 ** 64
    situ_b2: float = 2.0 ** 64
    rms_eps: float = 1e-5
    trunk_sigma: float = 0.02
    gate: np.ndarray = None
    bias: np.ndarray = None
    sh1: np.ndarray = None
    sh3: np.ndarray = None
    sh2: np.ndarray = None
    down: np.ndarray = None
    up: np.ndarray = None
    lnorm: np.ndarray = None
    _cache: dict = field(default_factory=dict)
    _held: dict = field(default_factory=dict)

    @property
    def XL(self):
        """The routed experts' width: the latent width, or H without a projection."""
        return self.latent if self.latent > 0 else self.H

    def __post_init__(self):
        H, E, I, SI = self.H, self.E, self.I, self.I * self.n_shared
        s, l = self.seed, self.layer
        self.gate = normal_f32(E * H, key(s, l, S_ROUTER), 0.0, self.router_sigma).reshape(E, H)
        if self.zipf_alpha > 0:
            self.bias = np.empty(E, np.float32)
            oracle().ko_zipf_bias(ptr(self.bias, F32P), E, key(s, l, S_BIAS), self.zipf_alpha,
                                  self.zipf_s)
        else:
            self.bias = normal_f32(E, key(s, l, S_BIAS), 0.0, self.bias_sigma)
        if SI > 0:
            self.sh1 = normal_bf16(SI * H, key(s, l, S_SH1), 0.0, self.shared_sigma).reshape(SI, H)
            self.sh3 = normal_bf16(SI * H, key(s, l, S_SH3), 0.0, self.shared_sigma).reshape(SI, H)
            self.sh2 = normal_bf16(H * SI, key(s, l, S_SH2), 0.0, self.shared_sigma).reshape(H, SI)
        if self.latent > 0:
            LT = self.latent
            self.down = normal_bf16(LT * H, key(s, l, S_DOWN), 0.0, self.trunk_sigma).reshape(LT, H)
            self.up = normal_bf16(H * LT, key(s, l, S_UP), 0.0, self.trunk_sigma).reshape(H, LT)
        if self.latent_norm:
            self.lnorm = normal_f32(self.XL, key(s, l, S_LNORM), 1.0, 0.1)

    def expert(self, e):
        """Expert e's six arrays in the reference's row-major layout (cached)."""
        if e in self._held:
            return self._held[e]
        if e in self._cache:
            return self._cache[e]
        H, I, s, l = self.XL, self.I, self.seed, self.layer
        d = {}
        for m, (pk, sk, R, Kc) in enumerate((("p1", "s1", I, H), ("p3", "s3", I, H),
                                             ("p2", "s2", H, I))):
            d[pk] = codes(R * Kc // 2, key(s, l, S_CODES, 3 * e + m)).reshape(R, Kc // 2)
            d[sk] = scales(R * Kc // 32, key(s, l, S_SCALES, 3 * e + m), self.scale_lo,
                           self.scale_hi).reshape(R, Kc // 32)
        if len(self._cache) > 64:
            self._cache.clear()
        self._cache[e] = d
        return d

    def hold(self, experts):
        """Generates these experts once and keeps them until release(): the cache of
        expert() keeps at most 64, which a check over many tokens would regenerate."""
        for e in experts:
            e = int(e)
            if e not in self._held:
                self._held[e] = self.expert(e)

    def release(self):
        self._held.clear()

    def x(self, T, bf16=True, stream_sub=0):
        """T tokens N(0,1); rounded to bf16 values (returned as fp32) when bf16."""
        v = normal_f32(T * self.H, key(self.seed, self.layer, S_X, stream_sub)).reshape(T, self.H)
        if bf16:
            v = bf16_to_f32(f32_to_bf16(v)).reshape(T, self.H)
        return v

    # ---- the oracle on this layer ------------------------------------------------
    def ko_cfg(self):
        return KoCfg(self.H, self.E, self.K, self.I, self.n_shared, self.renorm,
                     self.routed_scale, self.situ_b1, self.situ_b2, 32, self.latent,
                     self.latent_norm, self.rms_eps)

    def _weights(self, fail=None):
        keep = []

        def get(ctx, e, q):
            if fail is not None and e in fail:
                return -1
            d = self.expert(e)
            keep.append(d)
            for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
                setattr(q.contents, k, d[k].ctypes.data_as(U8P))
            return 0

        cb = GET_FN(get)
        w = KoWeights(ptr(self.gate, F32P), ptr(self.bias, F32P), cb, None,
                      vptr(self.sh1), vptr(self.sh3), vptr(self.sh2), vptr(self.down),
                      vptr(self.up), ptr(self.lnorm, F32P), 0)
        return w, cb, keep

    def oracle_moe(self, x, prefill=False, fail=None):
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        out = np.empty_like(x)
        idx = np.empty((T, self.K), np.int32)
        wt = np.empty((T, self.K), np.float32)
        cfg = self.ko_cfg()
        w, cb, keep = self._weights(fail)
        if prefill:
            ng = C.c_long(0)
            drops = oracle().ko_moe_prefill(ptr(out, F32P), ptr(x, F32P), T, C.byref(cfg),
                                            C.byref(w), ptr(idx, I32P), ptr(wt, F32P),
                                            C.byref(ng))
            return out, idx, wt, drops, ng.value
        drops = oracle().ko_moe(ptr(out, F32P), ptr(x, F32P), T, C.byref(cfg), C.byref(w),
                                ptr(idx, I32P), ptr(wt, F32P))
        return out, idx, wt, drops

    def oracle_moe_cache_only(self, x, res):
        """The oracle of cache-only (draft) routing over the experts res marks resident."""
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        out = np.empty_like(x)
        idx = np.empty((T, self.K), np.int32)
        wt = np.empty((T, self.K), np.float32)
        cfg = self.ko_cfg()
        w, cb, keep = self._weights(None)
        r = np.ascontiguousarray(res, np.int32)
        oracle().ko_moe_cache_only(ptr(out, F32P), ptr(x, F32P), T, C.byref(cfg), C.byref(w),
                                   ptr(r, I32P), ptr(idx, I32P), ptr(wt, F32P))
        return out, idx, wt

    def oracle_moe_mx(self, x, fail=None):
        """The oracle of the MXFP8-activation prefill mode (ko_moe_mx)."""
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        out = np.empty_like(x)
        idx = np.empty((T, self.K), np.int32)
        wt = np.empty((T, self.K), np.float32)
        cfg = self.ko_cfg()
        w, cb, keep = self._weights(fail)
        drops = oracle().ko_moe_mx(ptr(out, F32P), ptr(x, F32P), T, C.byref(cfg), C.byref(w),
                                   ptr(idx, I32P), ptr(wt, F32P))
        return out, idx, wt, drops

    def all_experts(self):
        return [self.expert(e) for e in range(self.E)]


def tiny(seed=0, **kw):
    """The reference-CPU-path configuration: H 256, 16 experts top-4, I 128, 1 shared."""
    return Layer(H=256, E=16, K=4, I=128, seed=seed, **kw)


def tiny_latent(seed=0, **kw):
    """A small LatentMoE layer: H 256, latent 128, 16 experts top-4, I 128, 2 shared,
    SiTU betas 4 and 25, the latent RMSNorm."""
    kw = {"routed_scale": 1.0, "n_shared": 2, "latent": 128, "latent_norm": 1,
          "situ_b1": 4.0, "situ_b2": 25.0, **kw}
    return Layer(H=256, E=16, K=4, I=128, seed=seed, **kw)


def k3(seed=0, **kw):
    """The K3 LatentMoE shape: H 7168, latent 3584, 896 experts top-16, I 3072, 2 shared
    bf16 experts, SiTU betas 4 and 25, the latent RMSNorm, routed_scale 1."""
    kw = {"routed_scale": 1.0, "n_shared": 2, "latent": 3584, "latent_norm": 1,
          "situ_b1": 4.0, "situ_b2": 25.0, **kw}
    return Layer(H=7168, E=896, K=16, I=3072, seed=seed, **kw)


def full(seed=0, **kw):
    """The K2-class shape: H 7168, 384 experts top-8, I 2048, 1 bf16 shared expert."""
    return Layer(H=7168, E=384, K=8, I=2048, seed=seed, **kw)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def rms_inv(ss, n, eps):
    """The reference's RMSNorm scale from a sum of squares (k3_ops.c:137)."""
    import math
    return np.float32(1.0 / math.sqrt(ss / n + eps))


def rms_window_row(n, eps, seed):
    """A float row whose sum of squares lies within 2^-44 relative of the preimage of a
    float rounding midpoint of the RMSNorm scale, so that a kernel summing the squares in
    another order than the reference's chain cannot prove its float scale from its own
    sum and must fall back to the chain.  Built from N(0, 1) entries, a coarse entry at
    column 0 and a fine one at column 1 (its square steps by about 2^-43) that together
    put the exact sum on the target."""
    import math
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    rest = math.fsum(float(v) * float(v) for v in x[2:])
    f0 = rms_inv(rest + 1.0, n, eps)
    f1 = np.nextafter(f0, np.float32(np.inf))
    m = (float(f0) + float(f1)) / 2.0
    R = n * (1.0 / (m * m) - eps) - rest          # the two entries' squares' target sum
    c = np.float32(math.sqrt(R - 2.0 ** -21))
    while float(c) * float(c) > R - 2.0 ** -22:
        c = np.nextafter(c, np.float32(0))
    f = np.float32(math.sqrt(R - float(c) * float(c)))
    x[0], x[1] = c, f
    ss = math.fsum(float(v) * float(v) for v in x)
    assert abs(ss - n * (1.0 / (m * m) - eps)) <= 2.0 ** -44 * ss, "window missed"
    return x
