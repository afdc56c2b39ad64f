"""The trunk's host layer (k3x_trunk.c) on the CPU, over a recording stand-in for the HIP
runtime (tests/mock/hip_mock.c): the workspace of calls past eight rows grows (at least
doubling) outside capture only; a call that would grow it on a stream under capture
returns K3X_E_SHAPE and launches nothing; an outgrown workspace is retired, not freed,
so a graph captured over it stays valid, and destroy frees every generation.  Both
product paths are covered: the library GEMM (fp32 rows split into the workspace, then two
bf16 GEMMs) and the dense kernel used where the library is absent."""
import ctypes as C
import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "kimi-k3-for-me_amd", "csrc")
K3X_E_SHAPE, K3X_E_NOMEM = -2, -4


@pytest.fixture(scope="module")
def mock(tmp_path_factory):
    if shutil.which("gcc") is None or not os.path.isdir("/opt/rocm/include/hip"):
        pytest.skip("gcc or the HIP headers are absent")
    out = str(tmp_path_factory.mktemp("trunkmock") / "libtrunkmock.so")
    subprocess.run(["gcc", "-O1", "-std=gnu99", "-shared", "-fPIC", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", os.path.join(CSRC, "k3x_trunk.c"),
                    os.path.join(HERE, "mock", "hip_mock.c"), "-o", out], check=True)
    lib = C.CDLL(out)
    vp = C.c_void_p
    lib.k3x_trunk_create.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.POINTER(vp)]
    lib.k3x_trunk_apply.argtypes = [vp, vp, C.c_int, vp, C.c_int, C.c_int, C.c_int, vp]
    lib.k3x_trunk_reserve.argtypes = [vp, C.c_int]
    lib.k3x_trunk_destroy.argtypes = [vp]
    lib.k3x_trunk_destroy.restype = None
    lib.mock_last_planes.restype = vp
    lib.mock_is_live.argtypes = [vp]
    return lib


@pytest.mark.parametrize("blas", [0, 1])
def test_workspace_growth_capture_and_retirement(mock, blas):
    mock.mock_reset()
    mock.mock_set_blas(blas)
    IN, OUT = 256, 32
    W = np.zeros((OUT, IN), np.uint16)
    t = C.c_void_p()
    assert mock.k3x_trunk_create(W.ctypes.data, IN, OUT, 0, C.byref(t)) == 0
    x = np.zeros((4096, IN), np.float32)          # never read by the stand-in
    y = np.zeros((4096, OUT), np.float32)
    base = mock.mock_mallocs()

    def apply(T):
        return mock.k3x_trunk_apply(t, y.ctypes.data, OUT, x.ctypes.data, 0, IN, T, None)

    assert apply(8) == 0 and mock.mock_mallocs() == base       # GEMV: no workspace
    assert apply(16) == 0 and mock.mock_mallocs() == base + 1
    p16 = mock.mock_last_planes()
    assert apply(20) == 0 and mock.mock_mallocs() == base + 2  # grows: at least doubles
    p32 = mock.mock_last_planes()
    assert p32 != p16 and mock.mock_is_live(p16)               # retired, not freed
    assert apply(32) == 0 and mock.mock_last_planes() == p32   # 32 rows fit the doubled one
    # under capture: a call within the workspace is captured, a larger one refused
    mock.mock_set_capturing(1)
    g = mock.mock_gemms()
    assert apply(30) == 0 and mock.mock_gemms() == g + 1
    assert apply(33) == K3X_E_SHAPE
    assert mock.mock_gemms() == g + 1 and mock.mock_mallocs() == base + 2
    mock.mock_set_capturing(0)
    # reserve outside capture; a capture of that size then runs in the reserved workspace
    assert mock.k3x_trunk_reserve(t, 200) == 0
    p200 = mock.mock_last_planes()
    mock.mock_set_capturing(1)
    assert apply(200) == 0
    p = mock.mock_last_planes()
    assert p != p32 and p != p16 and mock.mock_is_live(p32) and mock.mock_is_live(p16)
    mock.mock_set_capturing(0)
    # the library path: two GEMMs (hi, then lo accumulated) per product past 8 rows
    assert mock.mock_blas_calls() == (2 * mock.mock_gemms() if blas else 0)
    live = mock.mock_live()
    frees = mock.mock_frees()
    mock.k3x_trunk_destroy(t)
    assert mock.mock_live() == 0 and mock.mock_frees() == frees + live
    del p200


def test_workspace_generations_are_bounded(mock):
    mock.mock_reset()
    IN, OUT = 128, 16
    W = np.zeros((OUT, IN), np.uint16)
    t = C.c_void_p()
    assert mock.k3x_trunk_create(W.ctypes.data, IN, OUT, 0, C.byref(t)) == 0
    rcs = [mock.k3x_trunk_reserve(t, 9 << k) for k in range(18)]
    assert rcs[:17] == [0] * 17 and rcs[17] == K3X_E_NOMEM
    mock.k3x_trunk_destroy(t)
    assert mock.mock_live() == 0
