"""The decode kernels' per-workgroup trace (a layer made with K3X_TRACE=1): one record per
workgroup of each kernel, start before end, an XCD id below 8, and the call's results
unchanged by the tracing."""
import os

import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, say

pytestmark = pytest.mark.gpu


def test_decode_trace_records(torch, k3x):
    say("case: tiny layer, decode T=1 with the per-workgroup trace")
    L = synth.tiny(seed=51)
    os.environ["K3X_TRACE"] = "1"
    try:
        layer = bank_layer(k3x, L)
    finally:
        del os.environ["K3X_TRACE"]
    x = L.x(1, bf16=False, stream_sub=5)
    o, idx, _, _ = L.oracle_moe(x)
    out, i2, _ = dev_forward(torch, k3x, layer, x)
    assert np.array_equal(i2, idx) and synth.rel_l2(out, o) < 1e-3
    grids = [L.E, 1 + L.I * L.n_shared // 16 + L.K * (L.I // 16) // 4, L.H // 16]
    for k, g in enumerate(grids):
        t = layer.trace(k)
        assert t is not None and len(t) == g, (k, None if t is None else len(t), g)
        t = t.astype(np.int64)
        wg = t[:, 0] & 0x0FFFFFFF
        xcd = (t[:, 0] >> 28) & 15
        assert np.array_equal(wg, np.arange(g))
        assert np.all(xcd < 8)
        assert np.all(t[:, 2] >= t[:, 1])
    layer.close()
