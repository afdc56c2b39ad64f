"""The trunk's bf16 products on the device (include/k3x_trunk.h) against the oracle's
ko_matmul_bf16, which is bitwise the reference's k3_matmul_bf16 (tests/test_oracle.py):
Y[t*ldy + o] = W[o] . X[t*ldx] for the GEMV (T <= 8) and the GEMM (T > 8), fp32 and bf16
activations, padded row strides."""
import numpy as np
import pytest

import synth
from gpu_util import say
from oracle_lib import F32P, U16P, oracle, ptr

pytestmark = pytest.mark.gpu


def oracle_rows(W, X):
    out, inn = W.shape
    Y = np.empty((X.shape[0], out), np.float32)
    for t in range(X.shape[0]):
        xt = np.ascontiguousarray(X[t], np.float32)
        oracle().ko_matmul_bf16(ptr(Y[t], F32P), ptr(xt, F32P), ptr(W, U16P), inn, out)
    return Y


@pytest.mark.parametrize("inn,out,T,bf16", [
    (256, 64, 1, False), (7168, 1536, 3, False), (3584, 7168, 8, True),
    (1536, 3072, 9, False), (7168, 512, 64, True), (512, 7168, 300, False)])
def test_trunk_vs_oracle(torch, k3x, inn, out, T, bf16):
    say(f"case: trunk product in={inn} out={out} T={T} bf16={bf16}")
    rng = np.random.default_rng(inn + out + T)
    W = synth.f32_to_bf16((rng.standard_normal((out, inn)) * 0.03).astype(np.float32))
    X = rng.standard_normal((T, inn)).astype(np.float32)
    if bf16:
        X = synth.bf16_to_f32(synth.f32_to_bf16(X)).reshape(T, inn)
    tr = k3x.Trunk(W)
    xd = torch.from_numpy(X).cuda()
    if bf16:
        xd = xd.to(torch.bfloat16)
    yd = torch.empty((T, out), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    tr.apply(yd.data_ptr(), out, xd.data_ptr(), k3x.K3X_BF16 if bf16 else k3x.K3X_F32, inn, T, s)
    torch.cuda.synchronize()
    want = oracle_rows(W, X)
    err = synth.rel_l2(yd.cpu().numpy(), want)
    say(f"  rel_l2={err:.3e}")
    assert err < (1e-6 if bf16 else 2e-5)
    tr.close()


@pytest.mark.parametrize("T", [5, 40])
def test_trunk_strides_and_host_form(torch, k3x, T):
    """ldx > in and ldy > out (a sub-range of rows, k3_mmw_batch_ld): the padding of Y is
    left alone; the host-pointer form gives the same rows."""
    say(f"case: trunk product with row strides, T={T}")
    inn, out, ldx, ldy = 1024, 256, 1032, 300
    rng = np.random.default_rng(T)
    W = synth.f32_to_bf16((rng.standard_normal((out, inn)) * 0.05).astype(np.float32))
    Xp = rng.standard_normal((T, ldx)).astype(np.float32)
    tr = k3x.Trunk(W)
    xd = torch.from_numpy(Xp).cuda()
    yd = torch.full((T, ldy), 7.0, dtype=torch.float32, device="cuda")
    tr.apply(yd.data_ptr(), ldy, xd.data_ptr(), k3x.K3X_F32, ldx, T,
             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y = yd.cpu().numpy()
    assert np.all(y[:, out:] == 7.0)
    want = oracle_rows(W, Xp[:, :inn])
    assert synth.rel_l2(y[:, :out], want) < 2e-5
    yh = tr.apply_host(Xp[:, :inn])
    assert np.array_equal(yh, y[:, :out])
    tr.close()


def test_trunk_graph_capture_and_growth(torch, k3x):
    """A product of 40 rows captured after a reserve, replayed on new inputs; a larger
    call under capture is refused (K3X_E_SHAPE) without enqueuing; an eager call that
    outgrows the workspace afterwards leaves the captured graph valid (its workspace is
    retired, not freed): every replay equals the eager product of the same rows."""
    say("case: trunk GEMM captured after reserve, refused growth, replays after growth")
    inn, out, T = 1024, 512, 40
    rng = np.random.default_rng(77)
    W = synth.f32_to_bf16((rng.standard_normal((out, inn)) * 0.05).astype(np.float32))
    tr = k3x.Trunk(W)
    tr.reserve(T)
    xd = torch.empty((T, inn), dtype=torch.float32, device="cuda")
    yd = torch.empty((T, out), dtype=torch.float32, device="cuda")
    big_x = torch.zeros((4 * T, inn), dtype=torch.float32, device="cuda")
    big_y = torch.empty((4 * T, out), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    refused = None
    with torch.cuda.graph(g, stream=s):
        tr.apply(yd.data_ptr(), out, xd.data_ptr(), k3x.K3X_F32, inn, T, s.cuda_stream)
        try:
            tr.apply(big_y.data_ptr(), out, big_x.data_ptr(), k3x.K3X_F32, inn, 4 * T,
                     s.cuda_stream)
        except k3x.K3XError as e:
            refused = e
    torch.cuda.synchronize()
    assert refused is not None and refused.status == -2        # K3X_E_SHAPE
    for r in range(3):
        X = rng.standard_normal((T, inn)).astype(np.float32)
        xd.copy_(torch.from_numpy(X))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = yd.cpu().numpy()
        if r == 1:
            # outgrow the workspace eagerly between replays
            tr.apply(big_y.data_ptr(), out, big_x.data_ptr(), k3x.K3X_F32, inn, 4 * T)
            torch.cuda.synchronize()
        tr.apply(yd.data_ptr(), out, xd.data_ptr(), k3x.K3X_F32, inn, T)
        torch.cuda.synchronize()
        say(f"  replay {r}")
        assert np.array_equal(got, yd.cpu().numpy())
        assert synth.rel_l2(got, oracle_rows(W, X)) < 2e-5
    g.replay()
    torch.cuda.synchronize()
    assert np.array_equal(yd.cpu().numpy(), got)
    tr.close()
