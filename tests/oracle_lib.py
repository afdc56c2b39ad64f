"""ctypes view of the oracle (oracle/k3x_oracle.c) and of the compiled reference.

Test infrastructure only: the oracle checks device results.  The compiled reference
(oracle/_ref/libk3ref.so, built from the reference's own k3_ops.c) is optional and
only pins the oracle; tests that need it skip when it was not built.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "libk3x_oracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libk3ref.so")
REF_V4_SO = os.path.join(ROOT, "oracle", "_ref", "libk3ref_v4.so")

F32P = C.POINTER(C.c_float)
U8P = C.POINTER(C.c_uint8)
U16P = C.POINTER(C.c_uint16)
I32P = C.POINTER(C.c_int)


def ptr(a, t):
    return a.ctypes.data_as(t) if a is not None else None


class KoCfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_experts", C.c_int), ("topk", C.c_int),
                ("moe_inter", C.c_int), ("n_shared", C.c_int), ("renorm", C.c_int),
                ("routed_scale", C.c_float), ("situ_b1", C.c_float),
                ("situ_b2", C.c_float), ("group", C.c_int), ("latent", C.c_int),
                ("latent_norm", C.c_int), ("rms_eps", C.c_float)]


class KoExpert(C.Structure):
    _fields_ = [("p1", U8P), ("s1", U8P), ("p3", U8P), ("s3", U8P),
                ("p2", U8P), ("s2", U8P)]


GET_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.POINTER(KoExpert))


class KoWeights(C.Structure):
    _fields_ = [("gate", F32P), ("bias", F32P), ("get", GET_FN), ("ctx", C.c_void_p),
                ("sh1", C.c_void_p), ("sh3", C.c_void_p), ("sh2", C.c_void_p),
                ("down", C.c_void_p), ("up", C.c_void_p), ("latent_norm", F32P),
                ("trunk_f32", C.c_int), ("w1", F32P), ("w3", F32P), ("w2", F32P)]


class DrvCfg(C.Structure):
    """drv_cfg of oracle/ref_driver.c: the K3Cfg fields of the MoE block."""
    _fields_ = [("hidden", C.c_int), ("latent", C.c_int), ("n_experts", C.c_int),
                ("topk", C.c_int), ("inter", C.c_int), ("n_shared", C.c_int),
                ("renorm", C.c_int), ("latent_norm", C.c_int), ("routed_scale", C.c_float),
                ("rms_eps", C.c_float), ("situ_b1", C.c_float), ("situ_b2", C.c_float)]


def vptr(a):
    """Address of an array as a void pointer (None for None)."""
    return a.ctypes.data if a is not None else None


def _load(path):
    if not os.path.exists(path):
        return None
    return C.CDLL(path)


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        lib = _load(ORACLE_SO)
        if lib is None:
            raise RuntimeError("oracle not built: run `make -C oracle`")
        lib.ko_e2m1.restype = C.c_float
        lib.ko_e8m0.restype = C.c_float
        lib.ko_sigmoidf.restype = C.c_float
        lib.ko_sigmoidf.argtypes = [C.c_float]
        lib.ko_rmsnorm.argtypes = [F32P, F32P, F32P, C.c_int, C.c_float]
        lib.ko_situ_glu.argtypes = [F32P, F32P, C.c_int, C.c_float, C.c_float]
        lib.ko_router.argtypes = [I32P, F32P, F32P, F32P, F32P, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_float]
        lib.ko_matmul_mxfp4.argtypes = [F32P, F32P, U8P, U8P, C.c_int, C.c_int, C.c_int]
        lib.ko_mxfp4_dequant.argtypes = [F32P, U8P, U8P, C.c_int, C.c_int, C.c_int]
        lib.ko_matmul_bf16.argtypes = [F32P, F32P, U16P, C.c_int, C.c_int]
        lib.ko_matmul_f32.argtypes = [F32P, F32P, F32P, C.c_int, C.c_int]
        lib.ko_moe.restype = C.c_long
        lib.ko_moe.argtypes = [F32P, F32P, C.c_int, C.POINTER(KoCfg), C.POINTER(KoWeights),
                               I32P, F32P]
        lib.ko_moe_prefill.restype = C.c_long
        lib.ko_moe_prefill.argtypes = [F32P, F32P, C.c_int, C.POINTER(KoCfg),
                                       C.POINTER(KoWeights), I32P, F32P,
                                       C.POINTER(C.c_long)]
        lib.ko_e4m3.restype = C.c_float
        lib.ko_e4m3.argtypes = [C.c_int]
        lib.ko_e4m3_rne.argtypes = [C.c_float]
        lib.ko_mx8_scale.argtypes = [F32P, C.c_int]
        lib.ko_mx8_quant.argtypes = [U8P, U8P, F32P, C.c_int]
        lib.ko_mx8_dequant.argtypes = [C.POINTER(C.c_double), U8P, U8P, C.c_int]
        lib.ko_matmul_mx.argtypes = [F32P, U8P, U8P, U8P, U8P, C.c_int, C.c_int]
        lib.ko_moe_cache_only.restype = C.c_long
        lib.ko_moe_cache_only.argtypes = [F32P, F32P, C.c_int, C.POINTER(KoCfg),
                                          C.POINTER(KoWeights), I32P, I32P, F32P]
        lib.ko_moe_mx.restype = C.c_long
        lib.ko_moe_mx.argtypes = [F32P, F32P, C.c_int, C.POINTER(KoCfg), C.POINTER(KoWeights),
                                  I32P, F32P]
        lib.ko_attn_res.argtypes = [F32P, F32P, F32P, C.c_int, C.c_int, C.c_float]
        lib.ko_moe_half.restype = C.c_long
        lib.ko_moe_half.argtypes = [F32P, F32P, F32P, C.c_int, C.c_int, F32P, F32P, C.c_float,
                                    C.c_int, C.POINTER(KoCfg), C.POINTER(KoWeights)]
        lib.ko_moe_half_v.restype = C.c_long
        lib.ko_moe_half_v.argtypes = [F32P, F32P, F32P, C.c_int, I32P, C.c_int, F32P, F32P,
                                      C.c_float, C.c_int, C.POINTER(KoCfg),
                                      C.POINTER(KoWeights)]
        lib.ko_stack_step.restype = C.c_long
        lib.ko_stack_step.argtypes = [F32P, C.c_int, C.c_int, C.POINTER(KoCfg),
                                      C.POINTER(C.POINTER(KoWeights)),
                                      C.POINTER(F32P), C.c_float]
        lib.ko_mix64.restype = C.c_uint64
        lib.ko_mix64.argtypes = [C.c_uint64]
        lib.ko_key.restype = C.c_uint64
        lib.ko_key.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int]
        lib.ko_draw.restype = C.c_uint64
        lib.ko_draw.argtypes = [C.c_uint64, C.c_uint64]
        lib.ko_fill_normal_f32.argtypes = [F32P, C.c_size_t, C.c_uint64, C.c_double,
                                           C.c_double]
        lib.ko_fill_normal_bf16.argtypes = [U16P, C.c_size_t, C.c_uint64, C.c_double,
                                            C.c_double]
        lib.ko_fill_codes.argtypes = [U8P, C.c_size_t, C.c_uint64]
        lib.ko_fill_scales.argtypes = [U8P, C.c_size_t, C.c_uint64, C.c_int, C.c_int]
        lib.ko_zipf_bias.argtypes = [F32P, C.c_int, C.c_uint64, C.c_double, C.c_double]
        lib.ko_f32_to_bf16.restype = C.c_uint16
        lib.ko_f32_to_bf16.argtypes = [C.c_float]
        lib.ko_now.restype = C.c_double
        lib.ko_threads.restype = C.c_int
        _oracle = lib
    return _oracle


_ref = {}

AVX512 = ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")


def host_has_x86_64_v4():
    """The host CPU has the AVX-512 subsets x86-64-v4 requires (from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    return all(x in fl for x in AVX512)
    except OSError:
        pass
    return False


def ref(isa="x86-64-v3"):
    """The compiled reference, or None when oracle/_ref was not built: the x86-64-v3
    build (AVX2 + FMA), or with isa="x86-64-v4" the AVX-512 build (None where the
    host lacks AVX-512)."""
    path = REF_V4_SO if isa == "x86-64-v4" else REF_SO
    if isa == "x86-64-v4" and not host_has_x86_64_v4():
        return None
    if path not in _ref:
        lib = _load(path)
        if lib is None:
            return None
        lib.k3_router.argtypes = [I32P, F32P, F32P, F32P, F32P, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_float]
        lib.k3_matmul_mxfp4.argtypes = [F32P, F32P, U8P, U8P, C.c_int, C.c_int, C.c_int]
        lib.k3_matmul_bf16.argtypes = [F32P, F32P, U16P, C.c_int, C.c_int]
        lib.k3_matmul.argtypes = [F32P, F32P, F32P, C.c_int, C.c_int]
        lib.k3_situ_glu.argtypes = [F32P, F32P, C.c_int, C.c_float, C.c_float]
        lib.k3_rmsnorm.argtypes = [F32P, F32P, F32P, C.c_int, C.c_float]
        lib.refdrv_moe.restype = C.c_long
        lib.refdrv_moe.argtypes = [F32P, F32P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_float, C.c_int, F32P, F32P,
                                   C.POINTER(KoExpert), I32P, U16P, U16P, U16P, C.c_int,
                                   I32P, F32P, C.POINTER(C.c_long)]
        lib.refdrv_moe_cfg.restype = C.c_long
        lib.refdrv_moe_cfg.argtypes = [F32P, F32P, C.c_int, C.POINTER(DrvCfg), F32P, F32P,
                                       C.POINTER(KoExpert), I32P, C.c_void_p, C.c_void_p,
                                       F32P, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                       C.c_int, I32P, F32P, C.POINTER(C.c_long)]
        lib.k3_attn_res.argtypes = [F32P, F32P, F32P, C.c_int, C.c_int, C.c_float]
        lib.refdrv_moe_half_v.restype = C.c_long
        lib.refdrv_moe_half_v.argtypes = [F32P, F32P, F32P, C.c_int, I32P, C.c_int, F32P,
                                          F32P, C.c_float, C.c_int, C.POINTER(DrvCfg), F32P,
                                          F32P, C.POINTER(KoExpert), C.c_void_p, C.c_void_p,
                                          F32P, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.refdrv_k2_tokens.restype = C.c_long
        lib.refdrv_k2_tokens.argtypes = [F32P, F32P, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.c_int, C.c_int, C.c_float, C.c_int, F32P, F32P,
                                         C.POINTER(KoExpert), U16P, U16P, U16P, I32P, F32P]
        lib.refdrv_k2_prefill.restype = C.c_long
        lib.refdrv_k2_prefill.argtypes = lib.refdrv_k2_tokens.argtypes
        lib.refdrv_k2_norm_layer.restype = C.c_long
        lib.refdrv_k2_norm_layer.argtypes = [F32P, C.c_int, F32P, C.c_float, C.c_int,
                                             C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                             C.c_int, F32P, F32P, C.POINTER(KoExpert), U16P,
                                             U16P, U16P, I32P, F32P]
        _ref[path] = lib
    return _ref[path]
