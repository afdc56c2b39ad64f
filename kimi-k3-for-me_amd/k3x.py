"""Python view of libk3x (the MoE block for MI355X), through its C ABI.

Mirrors the reference's MoE interface (k3_moe / k3_moe_prefill, include/k3/k3.h:
629-637; K3Cfg MoE fields k3.h:94-102; K3ExpertQ k3.h:507-516) with a device-resident
layer handle.  Every call goes through lib/libk3x.so; there is no Python or CPU
fallback: when the library is missing or no gfx950 device is visible, calls raise.

Device pointers are plain integers (e.g. torch.Tensor.data_ptr()); streams are
integers too (torch.cuda.Stream.cuda_stream) or 0 for the null stream.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libk3x.so")

K3X_F32 = 0
K3X_BF16 = 1
# prefill arithmetic (k3x_moe_layer_set_prefill_mode)
K3X_PREFILL_EXACT = 0
K3X_PREFILL_MXFP8 = 1
DECODE_MAX_T = 8

(STREAM_ROUTER, STREAM_BIAS, STREAM_X, STREAM_SH1, STREAM_SH3, STREAM_SH2, STREAM_NORM,
 STREAM_DOWN, STREAM_UP, STREAM_LNORM) = range(10)
STREAM_CODES, STREAM_SCALES = 10, 11

# the C-ABI surface declared in include/k3x_moe.h
EXPORTS = [
    "k3x_strerror", "k3x_moe_layer_create", "k3x_moe_layer_destroy", "k3x_moe_layer_bytes",
    "k3x_moe_layer_read_expert", "k3x_moe_forward", "k3x_rmsnorm", "k3x_moe",
    "k3x_moe_prefill", "k3x_expert_drops", "k3x_synth_layer_create", "k3x_synth_key",
    "k3x_synth_normal_f32", "k3x_synth_normal_bf16", "k3x_moe_layer_set_timing",
    "k3x_moe_layer_last_ms", "k3x_stack_create", "k3x_stack_forward", "k3x_stack_destroy",
    "k3x_moe_layer_check", "k3x_moe_layer_set_route_wait",
    "k3x_attn_res", "k3x_moe_half", "k3x_attn_res_v", "k3x_moe_half_v",
    "k3x_moe_layer_reserve", "k3x_moe_layer_dequant",
    "k3x_moe_prefill_noalloc", "k3x_moe_layer_trace", "k3x_moe_layer_set_prefill_mode",
    "k3x_moe_layer_exact_count", "k3x_moe_layer_last_route", "k3x_moe_route",
    # include/k3x_store.h
    "k3x_store_open", "k3x_store_close", "k3x_store_count", "k3x_store_shards",
    "k3x_store_find", "k3x_store_read", "k3x_store_expert_ref", "k3x_store_expert_load",
    "k3x_store_src_create", "k3x_store_src_create_for", "k3x_store_src_destroy",
    "k3x_store_src_fetches",
    "k3x_moe_layer_create_from_store",
    "k3x_moe_layer_create_cached",
    "k3x_cache_stats",
    "k3x_cache_pin", "k3x_cache_getmany", "k3x_cache_resident", "k3x_moe_layer_set_cache_only",
    "k3x_moe_layer_create_cached_src", "k3x_cache_slots_fit",
    # include/k3x_trunk.h
    "k3x_trunk_create", "k3x_trunk_destroy", "k3x_trunk_apply", "k3x_trunk_apply_host",
    "k3x_trunk_reserve",
]

DT_U8, DT_BF16, DT_F16, DT_F32 = 1, 2, 3, 4


class K3XError(RuntimeError):
    def __init__(self, status, what):
        super().__init__(f"{what}: {strerror(status)} ({status})")
        self.status = status


class Cfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_experts", C.c_int), ("topk", C.c_int),
                ("moe_inter", C.c_int), ("n_shared", C.c_int), ("moe_renorm", C.c_int),
                ("routed_scale", C.c_float), ("group", C.c_int), ("latent", C.c_int),
                ("latent_norm", C.c_int), ("rms_eps", C.c_float), ("situ_b1", C.c_float),
                ("situ_b2", C.c_float)]


class ExpertQ(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("p1", "s1", "p3", "s3", "p2", "s2")]


class ExpertSrc(C.Structure):
    pass


GET_FN = C.CFUNCTYPE(C.c_int, C.POINTER(ExpertSrc), C.c_int, C.c_int, C.POINTER(ExpertQ))
GETMANY_FN = C.CFUNCTYPE(C.c_int, C.POINTER(ExpertSrc), C.c_int, C.POINTER(C.c_int), C.c_int)
RESIDENT_FN = C.CFUNCTYPE(C.c_int, C.POINTER(ExpertSrc), C.c_int, C.c_int, C.POINTER(ExpertQ))
# get and ctx, then the two optional members (NULL unless set)
ExpertSrc._fields_ = [("get", GET_FN), ("ctx", C.c_void_p), ("getmany", GETMANY_FN),
                      ("resident", RESIDENT_FN)]


class MoeW(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("bias", C.c_void_p), ("sh1", C.c_void_p),
                ("sh3", C.c_void_p), ("sh2", C.c_void_p), ("src", C.POINTER(ExpertSrc)),
                ("bank", C.POINTER(ExpertQ)), ("layer", C.c_int), ("down", C.c_void_p),
                ("up", C.c_void_p), ("latent_norm", C.c_void_p)]


class TensorInfo(C.Structure):
    _fields_ = [("shard", C.c_int), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_int64 * 4), ("off", C.c_int64), ("nbytes", C.c_int64)]


class QMat(C.Structure):
    _fields_ = [("p_off", C.c_int64), ("p_bytes", C.c_int64), ("s_off", C.c_int64),
                ("s_bytes", C.c_int64), ("rows", C.c_int), ("pcols", C.c_int),
                ("scols", C.c_int)]


class ExpertRef(C.Structure):
    _fields_ = [("layer", C.c_int), ("expert", C.c_int), ("shard", C.c_int),
                ("off", C.c_int64), ("nbytes", C.c_int64), ("contiguous", C.c_int),
                ("m", QMat * 3)]


class SynthSpec(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("layer", C.c_int), ("router_sigma", C.c_double),
                ("bias_sigma", C.c_double), ("zipf_alpha", C.c_double),
                ("zipf_s", C.c_double), ("scale_lo", C.c_int), ("scale_hi", C.c_int),
                ("shared_sigma", C.c_double), ("trunk_sigma", C.c_double)]


_lib = None


def lib():
    """Load libk3x.so (raises when it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libk3x not built ({LIB_PATH}); run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        vp, i, f = C.c_void_p, C.c_int, C.c_float
        L.k3x_strerror.restype = C.c_char_p
        L.k3x_strerror.argtypes = [i]
        L.k3x_moe_layer_create.argtypes = [C.POINTER(Cfg), C.POINTER(MoeW), i, C.POINTER(vp)]
        L.k3x_moe_layer_destroy.argtypes = [vp]
        L.k3x_moe_layer_destroy.restype = None
        L.k3x_moe_layer_bytes.argtypes = [vp]
        L.k3x_moe_layer_bytes.restype = C.c_size_t
        L.k3x_moe_layer_read_expert.argtypes = [vp, i] + [vp] * 6
        L.k3x_moe_layer_reserve.argtypes = [vp, i]
        L.k3x_moe_layer_set_prefill_mode.argtypes = [vp, i]
        L.k3x_moe_layer_dequant.argtypes = [vp, i, i, vp]
        L.k3x_moe_forward.argtypes = [vp, vp, vp, i, i, vp, vp, vp, vp]
        L.k3x_moe_prefill_noalloc.argtypes = [vp, vp, vp, i, i, vp, vp, vp, vp]
        L.k3x_moe_route.argtypes = [vp, vp, vp, vp, i, i, vp]
        L.k3x_moe_layer_trace.argtypes = [vp, i, vp, i]
        L.k3x_moe_layer_exact_count.argtypes = [vp, C.POINTER(i)]
        L.k3x_moe_layer_last_route.argtypes = [vp, i, vp, vp]
        L.k3x_rmsnorm.argtypes = [vp, vp, vp, i, i, f, vp]
        L.k3x_moe.argtypes = [vp, vp, vp, i, vp, vp]
        L.k3x_moe_prefill.argtypes = [vp, vp, vp, i, vp, vp]
        L.k3x_synth_layer_create.argtypes = [C.POINTER(Cfg), C.POINTER(SynthSpec), i,
                                             C.POINTER(vp)]
        L.k3x_synth_key.argtypes = [C.c_uint64, i, i, i]
        L.k3x_synth_key.restype = C.c_uint64
        L.k3x_synth_normal_f32.argtypes = [vp, C.c_size_t, C.c_uint64, C.c_double, C.c_double]
        L.k3x_synth_normal_f32.restype = None
        L.k3x_synth_normal_bf16.argtypes = [vp, C.c_size_t, C.c_uint64, C.c_double, C.c_double]
        L.k3x_synth_normal_bf16.restype = None
        L.k3x_moe_layer_set_timing.argtypes = [vp, i]
        L.k3x_moe_layer_check.argtypes = [vp]
        L.k3x_moe_layer_set_route_wait.argtypes = [vp, C.c_ulonglong, i]
        L.k3x_moe_layer_last_ms.argtypes = [vp, C.POINTER(C.c_float)]
        L.k3x_stack_create.argtypes = [C.POINTER(vp), C.POINTER(vp), i, f, i, C.POINTER(vp)]
        L.k3x_stack_forward.argtypes = [vp, vp, i, vp]
        L.k3x_stack_destroy.argtypes = [vp]
        L.k3x_stack_destroy.restype = None
        L.k3x_store_open.argtypes = [C.c_char_p, C.POINTER(vp)]
        L.k3x_store_close.argtypes = [vp]
        L.k3x_store_close.restype = None
        L.k3x_store_count.argtypes = [vp]
        L.k3x_store_shards.argtypes = [vp]
        L.k3x_store_find.argtypes = [vp, C.c_char_p, C.POINTER(TensorInfo)]
        L.k3x_store_read.argtypes = [vp, C.c_char_p, vp, C.c_int64]
        L.k3x_store_read.restype = C.c_int64
        L.k3x_store_expert_ref.argtypes = [vp, i, i, C.POINTER(ExpertRef)]
        L.k3x_store_expert_load.argtypes = [vp, C.POINTER(ExpertRef), vp]
        L.k3x_store_expert_load.restype = C.c_int64
        L.k3x_store_src_create.argtypes = [vp, C.POINTER(vp)]
        L.k3x_store_src_create_for.argtypes = [vp, i, i, C.POINTER(vp)]
        L.k3x_store_src_destroy.argtypes = [vp]
        L.k3x_store_src_destroy.restype = None
        L.k3x_store_src_fetches.argtypes = [vp]
        L.k3x_store_src_fetches.restype = C.c_long
        L.k3x_moe_layer_create_from_store.argtypes = [C.POINTER(Cfg), C.POINTER(MoeW), vp, i, i,
                                                      C.POINTER(vp)]
        L.k3x_moe_layer_create_cached.argtypes = [C.POINTER(Cfg), C.POINTER(MoeW), vp, i, i, i,
                                                  C.POINTER(vp)]
        L.k3x_cache_stats.argtypes = [vp, C.POINTER(CacheStat)]
        L.k3x_cache_pin.argtypes = [vp, i, i]
        L.k3x_cache_getmany.argtypes = [vp, C.POINTER(C.c_int), i]
        L.k3x_cache_resident.argtypes = [vp, i]
        L.k3x_moe_layer_set_cache_only.argtypes = [vp, i, C.c_void_p]
        L.k3x_moe_layer_create_cached_src.argtypes = [C.POINTER(Cfg), C.POINTER(MoeW), i, i,
                                                      C.POINTER(vp)]
        L.k3x_cache_slots_fit.argtypes = [C.POINTER(Cfg), i, C.c_double]
        L.k3x_attn_res.argtypes = [vp, vp, i, i, vp, vp, i, i, f, vp]
        L.k3x_moe_half.argtypes = [vp, vp, vp, vp, i, i, vp, vp, f, i, vp, vp]
        L.k3x_attn_res_v.argtypes = [vp, vp, i, vp, i, vp, vp, i, i, f, vp]
        L.k3x_moe_half_v.argtypes = [vp, vp, vp, vp, i, vp, i, vp, vp, f, i, vp, vp]
        L.k3x_trunk_create.argtypes = [vp, i, i, i, C.POINTER(vp)]
        L.k3x_trunk_destroy.argtypes = [vp]
        L.k3x_trunk_destroy.restype = None
        L.k3x_trunk_apply.argtypes = [vp, vp, i, vp, i, i, i, vp]
        L.k3x_trunk_apply_host.argtypes = [vp, vp, vp, i]
        L.k3x_trunk_reserve.argtypes = [vp, i]
        _lib = L
    return _lib


def strerror(status):
    try:
        return lib().k3x_strerror(status).decode()
    except RuntimeError:
        return "libk3x not loaded"


def _check(rc, what):
    if rc < 0:
        raise K3XError(rc, what)
    return rc


def cache_slots_fit(cfg, device=0, fraction=0.75):
    """k3x_cache_slots_fit: expert slots that fit in that fraction of free device memory."""
    return _check(lib().k3x_cache_slots_fit(C.byref(cfg), device, fraction), "k3x_cache_slots_fit")


def expert_drops():
    return C.c_long.in_dll(lib(), "k3x_expert_drops").value


def attn_res(h, blocks, maxb, nb, pref, fold, n, T, eps=1e-5, stream=0):
    """Block attention-residual aggregation on device pointers (k3x_attn_res)."""
    _check(lib().k3x_attn_res(h, blocks or None, maxb, nb, pref, fold, n, T, eps,
                              stream or None), "k3x_attn_res")


def attn_res_v(h, blocks, maxb, nbv, nbs, pref, fold, n, T, eps=1e-5, stream=0):
    """The same with row t's block count nbv[t * nbs] read on the device (nbv a device
    int32 pointer; k3x_attn_res_v)."""
    _check(lib().k3x_attn_res_v(h, blocks or None, maxb, nbv, nbs, pref, fold, n, T, eps,
                                stream or None), "k3x_attn_res_v")


def make_cfg(hidden, n_experts, topk, moe_inter, n_shared=1, moe_renorm=1, routed_scale=2.5,
             group=32, latent=0, latent_norm=0, rms_eps=1e-5, situ_b1=0.0, situ_b2=0.0):
    """K3Cfg's MoE fields.  latent > 0 selects the LatentMoE form; betas of 0 (or 2^64)
    leave SiTU uncapped (SwiGLU)."""
    return Cfg(hidden, n_experts, topk, moe_inter, n_shared, moe_renorm, routed_scale, group,
               latent, latent_norm, rms_eps, situ_b1, situ_b2)


def _vp(a):
    return None if a is None else a.ctypes.data


def _supplier(get, getmany=None):
    """A k3x_expert_src over Python callables: get(layer, expert) -> dict of the six
    uint8 arrays (p1, s1, p3, s3, p2, s2) or None for a failed fetch; getmany(layer,
    experts) -> how many are now resident (optional).  Returns the struct and a dict
    that keeps the callbacks and the last expert's arrays alive: hold it as long as the
    library may call the supplier."""
    hold = {}

    def _get(src, lay, e, out):
        ex = get(lay, e)
        if ex is None:
            return -1
        arrs = {k: np.ascontiguousarray(ex[k], dtype=np.uint8)
                for k in ("p1", "s1", "p3", "s3", "p2", "s2")}
        hold["cur"] = arrs
        for k, a in arrs.items():
            setattr(out.contents, k, a.ctypes.data)
        return 0

    hold["get"] = GET_FN(_get)
    src = ExpertSrc(hold["get"], None)
    if getmany is not None:
        def _getmany(src_, lay, ex, n):
            return int(getmany(lay, [ex[i] for i in range(n)]))
        hold["getmany"] = GETMANY_FN(_getmany)
        src.getmany = hold["getmany"]
    hold["src"] = src
    return src, hold


class MoELayer:
    """A device-resident MoE layer (k3x_moe_layer)."""

    def __init__(self, handle, cfg):
        self.h = C.c_void_p(handle)
        self.cfg = cfg

    # -- construction -------------------------------------------------------------
    @classmethod
    def from_bank(cls, cfg, gate, bias, experts, sh1=None, sh3=None, sh2=None, device=0,
                  down=None, up=None, latent_norm=None):
        """experts: list of dicts with numpy uint8 arrays p1,s1,p3,s3,p2,s2; down/up bf16
        (uint16) and latent_norm fp32 numpy arrays for a latent layer."""
        keep = [gate, bias, sh1, sh3, sh2, down, up, latent_norm]
        bank = (ExpertQ * cfg.n_experts)()
        for e, ex in enumerate(experts):
            for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
                arr = np.ascontiguousarray(ex[k], dtype=np.uint8)
                keep.append(arr)
                setattr(bank[e], k, arr.ctypes.data)
        w = MoeW(_vp(gate), _vp(bias), _vp(sh1), _vp(sh3), _vp(sh2), None,
                 C.cast(bank, C.POINTER(ExpertQ)), 0, _vp(down), _vp(up), _vp(latent_norm))
        h = C.c_void_p()
        _check(lib().k3x_moe_layer_create(C.byref(cfg), C.byref(w), device, C.byref(h)),
               "k3x_moe_layer_create")
        return cls(h.value, cfg)

    @classmethod
    def from_source(cls, cfg, gate, bias, get, sh1=None, sh3=None, sh2=None, layer=0,
                    device=0, down=None, up=None, latent_norm=None, getmany=None):
        """get(layer, expert) -> dict of numpy arrays, or None for a failed fetch;
        getmany(layer, experts) -> how many are now resident (optional)."""
        src, _hold = _supplier(get, getmany)
        w = MoeW(_vp(gate), _vp(bias), _vp(sh1), _vp(sh3), _vp(sh2), C.pointer(src), None,
                 layer, _vp(down), _vp(up), _vp(latent_norm))
        h = C.c_void_p()
        _check(lib().k3x_moe_layer_create(C.byref(cfg), C.byref(w), device, C.byref(h)),
               "k3x_moe_layer_create")
        return cls(h.value, cfg)

    @classmethod
    def from_source_cached(cls, cfg, gate, bias, get, nslot, sh1=None, sh3=None, sh2=None,
                           layer=0, device=0, down=None, up=None, latent_norm=None,
                           getmany=None):
        """An HBM expert cache of nslot slots whose misses come through get (and getmany)
        as in from_source (k3x_moe_layer_create_cached_src); the callbacks are kept alive
        with the layer."""
        src, hold = _supplier(get, getmany)
        w = MoeW(_vp(gate), _vp(bias), _vp(sh1), _vp(sh3), _vp(sh2), C.pointer(src), None,
                 layer, _vp(down), _vp(up), _vp(latent_norm))
        h = C.c_void_p()
        _check(lib().k3x_moe_layer_create_cached_src(C.byref(cfg), C.byref(w), nslot, device,
                                                     C.byref(h)),
               "k3x_moe_layer_create_cached_src")
        layer_ = cls(h.value, cfg)
        layer_._hold = hold
        return layer_

    @classmethod
    def from_store(cls, cfg, gate, bias, store, layer, sh1=None, sh3=None, sh2=None, device=0,
                   down=None, up=None, latent_norm=None):
        """Routed experts streamed from a Store (k3x_moe_layer_create_from_store); the
        other weights as numpy arrays."""
        w = MoeW(_vp(gate), _vp(bias), _vp(sh1), _vp(sh3), _vp(sh2), None, None, layer,
                 _vp(down), _vp(up), _vp(latent_norm))
        h = C.c_void_p()
        _check(lib().k3x_moe_layer_create_from_store(C.byref(cfg), C.byref(w), store.h, layer,
                                                     device, C.byref(h)),
               "k3x_moe_layer_create_from_store")
        return cls(h.value, cfg)

    @classmethod
    def from_store_cached(cls, cfg, gate, bias, store, layer, nslot, sh1=None, sh3=None,
                          sh2=None, device=0, down=None, up=None, latent_norm=None):
        """A layer with an HBM expert cache of nslot slots over a Store
        (k3x_moe_layer_create_cached); decode calls only."""
        w = MoeW(_vp(gate), _vp(bias), _vp(sh1), _vp(sh3), _vp(sh2), None, None, layer,
                 _vp(down), _vp(up), _vp(latent_norm))
        h = C.c_void_p()
        _check(lib().k3x_moe_layer_create_cached(C.byref(cfg), C.byref(w), store.h, layer,
                                                 nslot, device, C.byref(h)),
               "k3x_moe_layer_create_cached")
        obj = cls(h.value, cfg)
        obj.store = store                       # the cache reads misses from it
        return obj

    def cache_stats(self):
        """k3x_cache_stats as a dict."""
        st = CacheStat()
        _check(lib().k3x_cache_stats(self.h, C.byref(st)), "k3x_cache_stats")
        return {f: int(getattr(st, f)) for f, _ in CacheStat._fields_}

    def cache_pin(self, expert, pin=True):
        _check(lib().k3x_cache_pin(self.h, expert, 1 if pin else 0), "k3x_cache_pin")

    def cache_getmany(self, experts):
        """k3x_cache_getmany: experts made resident together; returns how many are."""
        a = (C.c_int * len(experts))(*[int(e) for e in experts])
        return _check(lib().k3x_cache_getmany(self.h, a, len(experts)), "k3x_cache_getmany")

    def cache_resident(self, expert):
        return _check(lib().k3x_cache_resident(self.h, expert), "k3x_cache_resident")

    def set_cache_only(self, on, resident=None):
        """Cache-only (draft) routing over the experts resident[e] != 0 marks (numpy array
        of n_experts), or over the layer's own residency when resident is None."""
        keep = None
        if resident is not None:
            keep = np.ascontiguousarray(np.asarray(resident) != 0, dtype=np.uint8)
        _check(lib().k3x_moe_layer_set_cache_only(self.h, 1 if on else 0,
                                                  keep.ctypes.data if keep is not None else None),
               "k3x_moe_layer_set_cache_only")

    @classmethod
    def synthetic(cls, cfg, seed=0, layer=0, router_sigma=0.02, bias_sigma=0.1, zipf_alpha=0.0,
                  zipf_s=1.1, scale_lo=121, scale_hi=125, shared_sigma=0.02, device=0,
                  trunk_sigma=0.02):
        spec = SynthSpec(seed, layer, router_sigma, bias_sigma, zipf_alpha, zipf_s, scale_lo,
                         scale_hi, shared_sigma, trunk_sigma)
        h = C.c_void_p()
        _check(lib().k3x_synth_layer_create(C.byref(cfg), C.byref(spec), device, C.byref(h)),
               "k3x_synth_layer_create")
        return cls(h.value, cfg)

    def close(self):
        if self.h:
            lib().k3x_moe_layer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- calls --------------------------------------------------------------------
    def nbytes(self):
        return lib().k3x_moe_layer_bytes(self.h)

    def set_prefill_mode(self, mode):
        """K3X_PREFILL_EXACT (default) or the opt-in K3X_PREFILL_MXFP8."""
        _check(lib().k3x_moe_layer_set_prefill_mode(self.h, mode), "k3x_moe_layer_set_prefill_mode")

    def reserve(self, max_T):
        """Prefill buffers for calls of up to max_T tokens (needed before capturing one)."""
        _check(lib().k3x_moe_layer_reserve(self.h, max_T), "k3x_moe_layer_reserve")

    def forward(self, out_ptr, x_ptr, T, x_dtype=K3X_F32, resid_ptr=0, idx_ptr=0, wt_ptr=0,
                stream=0):
        """Device pointers (ints); asynchronous on `stream`."""
        _check(lib().k3x_moe_forward(self.h, out_ptr, x_ptr, x_dtype, T, resid_ptr or None,
                                     idx_ptr or None, wt_ptr or None, stream or None),
               "k3x_moe_forward")

    def route(self, idx_ptr, wt_ptr, x_ptr, T, x_dtype=K3X_F32, stream=0):
        """k3x_moe_route: every token's experts and weights (device pointers; asynchronous
        on `stream`)."""
        _check(lib().k3x_moe_route(self.h, idx_ptr, wt_ptr, x_ptr, x_dtype, T, stream or None),
               "k3x_moe_route")

    def prefill_noalloc(self, out_ptr, x_ptr, T, x_dtype=K3X_F32, resid_ptr=0, idx_ptr=0,
                        wt_ptr=0, stream=0):
        """k3x_moe_prefill_noalloc: the prefill path with its buffers in the static device
        array (device pointers; asynchronous on `stream`)."""
        _check(lib().k3x_moe_prefill_noalloc(self.h, out_ptr, x_ptr, x_dtype, T,
                                             resid_ptr or None, idx_ptr or None,
                                             wt_ptr or None, stream or None),
               "k3x_moe_prefill_noalloc")

    def moe(self, x, prefill=False):
        """Host call with k3_moe semantics: returns (out, idx_last, wt_last)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        out = np.empty_like(x)
        idx = np.zeros(self.cfg.topk, np.int32)
        wt = np.zeros(self.cfg.topk, np.float32)
        fn = lib().k3x_moe_prefill if prefill else lib().k3x_moe
        _check(fn(self.h, out.ctypes.data, x.ctypes.data, T, idx.ctypes.data, wt.ctypes.data),
               "k3x_moe")
        return out, idx, wt

    def read_expert(self, e):
        """Expert e in the reference's row-major layout; its width is the latent width in
        the latent form."""
        H = self.cfg.latent if self.cfg.latent > 0 else self.cfg.hidden
        I = self.cfg.moe_inter
        d = {"p1": np.empty((I, H // 2), np.uint8), "s1": np.empty((I, H // 32), np.uint8),
             "p3": np.empty((I, H // 2), np.uint8), "s3": np.empty((I, H // 32), np.uint8),
             "p2": np.empty((H, I // 2), np.uint8), "s2": np.empty((H, I // 32), np.uint8)}
        _check(lib().k3x_moe_layer_read_expert(self.h, e, *[d[k].ctypes.data for k in
                                                          ("p1", "s1", "p3", "s3", "p2", "s2")]),
               "k3x_moe_layer_read_expert")
        return d

    def dequant(self, e, m):
        """Matrix m (0 gate, 1 up, 2 down) of expert e as the device dequantises it
        (fp32 [rows][width])."""
        X = self.cfg.latent if self.cfg.latent > 0 else self.cfg.hidden
        I = self.cfg.moe_inter
        out = np.empty((X, I) if m == 2 else (I, X), np.float32)
        _check(lib().k3x_moe_layer_dequant(self.h, e, m, out.ctypes.data),
               "k3x_moe_layer_dequant")
        return out

    def moe_half(self, h, pref, blocks, maxb, nb, fold, post_norm, eps, T, hin, stream=0):
        """The MoE half of a decoder layer on device pointers (k3x_moe_half)."""
        _check(lib().k3x_moe_half(self.h, h, pref, blocks or None, maxb, nb, fold, post_norm,
                                  eps, T, hin, stream or None), "k3x_moe_half")

    def moe_half_v(self, h, pref, blocks, maxb, nbv, nbs, fold, post_norm, eps, T, hin,
                   stream=0):
        """The MoE half with row t's block count nbv[t * nbs] read on the device
        (k3x_moe_half_v)."""
        _check(lib().k3x_moe_half_v(self.h, h, pref, blocks or None, maxb, nbv, nbs, fold,
                                    post_norm, eps, T, hin, stream or None), "k3x_moe_half_v")

    def check(self):
        """Raise if a decode call since the last check had a workgroup give up waiting for
        the published selection (K3X_E_WAIT)."""
        _check(lib().k3x_moe_layer_check(self.h), "k3x_moe_layer_check")

    def set_route_wait(self, ticks, publish=True):
        """Failure injection: bound of the decode wait in 100 MHz ticks; publish=False
        withholds the selection's flag (calls made so are not valid)."""
        _check(lib().k3x_moe_layer_set_route_wait(self.h, ticks, 1 if publish else 0),
               "k3x_moe_layer_set_route_wait")

    def trace(self, kernel, max_wg=1 << 16):
        """Per-workgroup trace of decode kernel 0/1/2 of the last call ([n][3] uint64: id |
        XCD << 28 | hardware ids << 32, start, end at 100 MHz), or None (a layer made
        without K3X_TRACE=1)."""
        buf = np.zeros((max_wg, 3), np.uint64)
        n = _check(lib().k3x_moe_layer_trace(self.h, kernel, buf.ctypes.data, max_wg),
                   "k3x_moe_layer_trace")
        return buf[:n] if n else None

    def exact_count(self):
        """How many (token, expert) router logits the last decode-path selection worked
        out again as the reference's sequential chain (k3x_moe_layer_exact_count)."""
        n = C.c_int(0)
        _check(lib().k3x_moe_layer_exact_count(self.h, C.byref(n)), "k3x_moe_layer_exact_count")
        return n.value

    def last_route(self, T):
        """The last decode-path call's routing: (idx [T][K] int32, wt [T][K] float32)
        (k3x_moe_layer_last_route)."""
        K = self.cfg.topk
        idx = np.empty((T, K), np.int32)
        wt = np.empty((T, K), np.float32)
        _check(lib().k3x_moe_layer_last_route(self.h, T, idx.ctypes.data, wt.ctypes.data),
               "k3x_moe_layer_last_route")
        return idx, wt

    def set_timing(self, on):
        _check(lib().k3x_moe_layer_set_timing(self.h, 1 if on else 0), "set_timing")

    def last_ms(self):
        ms = (C.c_float * 8)()
        n = _check(lib().k3x_moe_layer_last_ms(self.h, ms), "last_ms")
        return [ms[i] for i in range(n)]


def rmsnorm(y_ptr, x_ptr, w_ptr, n, T, eps, stream=0):
    _check(lib().k3x_rmsnorm(y_ptr, x_ptr, w_ptr, n, T, eps, stream or None), "k3x_rmsnorm")


def synth_key(seed, layer, stream, sub=0):
    return lib().k3x_synth_key(seed, layer, stream, sub)


def synth_normal_f32(n, key, mu=0.0, sigma=1.0):
    a = np.empty(n, np.float32)
    lib().k3x_synth_normal_f32(a.ctypes.data, n, key, mu, sigma)
    return a


def synth_normal_bf16(n, key, mu=0.0, sigma=1.0):
    a = np.empty(n, np.uint16)
    lib().k3x_synth_normal_bf16(a.ctypes.data, n, key, mu, sigma)
    return a


class Stack:
    """Consecutive layers' MoE halves, h = h + MoE_l(RMSNorm_l(h)), replayed from a HIP
    graph (k3x_stack).  Layers and norm weights are borrowed: keep them alive."""

    def __init__(self, layers, norm_ptrs, eps=1e-5, max_T=1):
        n = len(layers)
        la = (C.c_void_p * n)(*[l.h.value for l in layers])
        na = (C.c_void_p * n)(*norm_ptrs)
        h = C.c_void_p()
        _check(lib().k3x_stack_create(la, na, n, eps, max_T, C.byref(h)), "k3x_stack_create")
        self.h = h
        self.layers = list(layers)

    def forward(self, h_ptr, T, stream=0):
        """h (device fp32 [T][hidden]) updated in place, asynchronously on `stream`."""
        _check(lib().k3x_stack_forward(self.h, h_ptr, T, stream or None), "k3x_stack_forward")

    def close(self):
        if self.h:
            lib().k3x_stack_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CacheStat(C.Structure):
    """k3x_cache_stat (include/k3x_store.h)."""
    _fields_ = [("nslot", C.c_int), ("resident", C.c_int), ("hits", C.c_ulonglong),
                ("misses", C.c_ulonglong), ("evictions", C.c_ulonglong),
                ("bytes_read", C.c_ulonglong)]


class Store:
    """A directory of safetensors shards (include/k3x_store.h), indexed by tensor name."""

    def __init__(self, path):
        self.h = C.c_void_p()
        _check(lib().k3x_store_open(os.fsencode(path), C.byref(self.h)), "k3x_store_open")

    def close(self):
        if self.h:
            lib().k3x_store_close(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def count(self):
        return lib().k3x_store_count(self.h)

    def shards(self):
        return lib().k3x_store_shards(self.h)

    def find(self, name):
        t = TensorInfo()
        if lib().k3x_store_find(self.h, name.encode(), C.byref(t)) != 0:
            return None
        return t

    def read(self, name):
        t = self.find(name)
        if t is None:
            raise K3XError(-1, f"k3x_store_read {name}")
        buf = np.empty(t.nbytes, np.uint8)
        _check(int(lib().k3x_store_read(self.h, name.encode(), buf.ctypes.data, t.nbytes)),
               "k3x_store_read")
        return buf

    def expert_ref(self, layer, expert):
        r = ExpertRef()
        _check(lib().k3x_store_expert_ref(self.h, layer, expert, C.byref(r)),
               "k3x_store_expert_ref")
        return r

    def expert_load(self, layer, expert):
        """(ref, bytes of the expert's run in the ref's layout)."""
        r = self.expert_ref(layer, expert)
        buf = np.empty(r.nbytes, np.uint8)
        _check(int(lib().k3x_store_expert_load(self.h, C.byref(r), buf.ctypes.data)),
               "k3x_store_expert_load")
        return r, buf


class Trunk:
    """A bf16 trunk matrix on the device (include/k3x_trunk.h): k3_mmw_batch_ld."""

    def __init__(self, W, device=0):
        W = np.ascontiguousarray(W, np.uint16)
        self.out, self.inn = W.shape
        self.h = C.c_void_p()
        _check(lib().k3x_trunk_create(W.ctypes.data, self.inn, self.out, device,
                                      C.byref(self.h)), "k3x_trunk_create")

    def close(self):
        if self.h:
            lib().k3x_trunk_destroy(self.h)
            self.h = C.c_void_p()

    def reserve(self, max_T):
        """Grow the workspace for calls of up to max_T rows (before a graph capture)."""
        _check(lib().k3x_trunk_reserve(self.h, max_T), "k3x_trunk_reserve")

    def apply(self, y, ldy, x, x_dtype, ldx, T, stream=0):
        """Device pointers: Y[t*ldy + o] = W[o] . X[t*ldx] for t < T."""
        _check(lib().k3x_trunk_apply(self.h, y, ldy, x, x_dtype, ldx, T, stream or None),
               "k3x_trunk_apply")

    def apply_host(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], self.out), np.float32)
        _check(lib().k3x_trunk_apply_host(self.h, y.ctypes.data, x.ctypes.data, x.shape[0]),
               "k3x_trunk_apply_host")
        return y
