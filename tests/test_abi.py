"""The C ABI: the library loads, exports every symbol include/k3x_moe.h declares,
validates arguments before touching a device, and its synthetic-layer generator is the
oracle's bit for bit (CPU only; no compute calls)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared():
    txt = "".join(open(h).read() for h in HEADERS)
    funcs = set(re.findall(r"\b(k3x_\w+)\s*\(", txt))
    data = set(re.findall(r"extern\s+long\s+(k3x_\w+)", txt))
    return funcs | data


def test_exports_every_declared_symbol(k3x):
    lib = k3x.lib()
    names = declared()
    assert len(names) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", k3x.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TBD]\s+(k3x_\w+)", out))
    missing = names - exported
    assert not missing, missing
    for n in names:
        getattr(lib, n)
    assert set(k3x.EXPORTS) <= names


def test_header_compiles_as_c_and_cxx(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "k3x_moe.h"\n#include "k3x_store.h"\n#include "k3x_trunk.h"\nint main(void){return K3X_OK;}\n')
    inc = os.path.join(ROOT, "include")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", inc, str(src)],
                   check=True)
    subprocess.run(["g++", "-x", "c++", "-Wall", "-Werror", "-fsyntax-only", "-I", inc, str(src)],
                   check=True)


def test_strerror(k3x):
    assert k3x.strerror(0) == "ok"
    assert "shape" in k3x.strerror(-2)
    assert "unknown" in k3x.strerror(-99)


@pytest.mark.parametrize("bad", [
    dict(hidden=250), dict(moe_inter=100), dict(group=16), dict(topk=0), dict(topk=65),
    dict(n_experts=2000), dict(topk=20, n_experts=16), dict(latent=100), dict(latent=-128),
])
def test_create_rejects_bad_cfg_before_device(k3x, bad):
    kw = dict(hidden=256, n_experts=16, topk=4, moe_inter=128)
    kw.update(bad)
    cfg = k3x.make_cfg(**kw)
    h = C.c_void_p()
    spec = k3x.SynthSpec(0, 0, 0.02, 0.1, 0.0, 1.1, 121, 125, 0.02)
    rc = k3x.lib().k3x_synth_layer_create(C.byref(cfg), C.byref(spec), 0, C.byref(h))
    assert rc == -2 and not h.value


@pytest.mark.parametrize("inn,out", [(100, 64), (256, 40), (0, 16)])
def test_trunk_rejects_bad_shapes_before_device(k3x, inn, out):
    W = np.zeros(max(inn * out, 1), np.uint16)
    h = C.c_void_p()
    rc = k3x.lib().k3x_trunk_create(W.ctypes.data, inn, out, 0, C.byref(h))
    assert rc in (-1, -2) and not h.value


def test_null_arguments(k3x):
    lib = k3x.lib()
    assert lib.k3x_moe_forward(None, None, None, 0, 1, None, None, None, None) == -1
    assert lib.k3x_moe(None, None, None, 1, None, None) == -1
    assert lib.k3x_moe_layer_create(None, None, 0, None) == -1
    assert lib.k3x_rmsnorm(None, None, None, 8, 1, 1e-5, None) == -1
    assert lib.k3x_moe_route(None, None, None, None, 0, 1, None) == -1


def test_synth_generator_matches_oracle(k3x):
    for (seed, layer, stream, sub) in ((0, 0, 0, 0), (7, 3, 5, 2), (123456789, 1, 11, 1151)):
        assert k3x.synth_key(seed, layer, stream, sub) == synth.key(seed, layer, stream, sub)
    k = synth.key(3, 1, 0)
    assert np.array_equal(k3x.synth_normal_f32(100003, k, 0.0, 0.02).view(np.uint32),
                          synth.normal_f32(100003, k, 0.0, 0.02).view(np.uint32))
    assert np.array_equal(k3x.synth_normal_bf16(70001, k, 0.0, 0.02),
                          synth.normal_bf16(70001, k, 0.0, 0.02))


def test_integration_adapter_compiles_against_reference_header(tmp_path):
    """The reference-side binding (k3x_ref_adapter.c) compiles against the
    reference's own k3.h and this library's header (build check only)."""
    if not os.path.isdir("/root/reference/include/k3"):
        pytest.skip("reference tree absent")
    adapter = os.path.join(ROOT, "kimi-k3-for-me_amd", "csrc", "k3x_ref_adapter.c")
    subprocess.run(["gcc", "-std=gnu99", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                    "-I", "/root/reference/include/k3", "-I", os.path.join(ROOT, "include"),
                    adapter], check=True)
