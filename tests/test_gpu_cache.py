"""The HBM expert cache's concurrent misses (k3x_cache_getmany, the misses of a call read
together), prefill calls on a cached layer, and cache-only (draft) routing
(k3x_moe_layer_set_cache_only, K3MoeW.cache_only: k3_ops.c:1884-1926), through the C ABI.

Cache-only outputs are checked against ko_moe_cache_only, which is bitwise the compiled
reference's k3_moe with cache_only set (test_oracle_cache.py): indices exact, weights to
float rounding, outputs within the parity bar."""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, layer_cfg, say
from test_gpu_store import run_bytes, write_layer

pytestmark = pytest.mark.gpu

TOL = 1e-3


def cached(k3x, st, L, layer, nslot):
    return k3x.MoELayer.from_store_cached(layer_cfg(k3x, L), L.gate, L.bias, st, layer, nslot,
                                          L.sh1, L.sh3, L.sh2, down=L.down, up=L.up,
                                          latent_norm=L.lnorm)


def decode_chunks(torch, k3x, layer, x):
    outs, idxs = [], []
    for t0 in range(0, x.shape[0], 8):
        o, i, _ = dev_forward(torch, k3x, layer, x[t0:t0 + 8])
        outs.append(o)
        idxs.append(i)
    return np.concatenate(outs), np.concatenate(idxs)


def test_cache_getmany_reads_together(torch, k3x, tmp_path):
    """Ten experts made resident in one call (more than the eight read at once): all
    resident, counted as ten misses of one run each; a second call over five of them and
    three new ones counts five hits' worth of no reads and three misses; more experts than
    slots is K3X_E_SHAPE; the layer then computes as the resident one, bit for bit."""
    say("case: k3x_cache_getmany over 10 then 8 experts, 12 slots")
    L = synth.Layer(H=256, E=24, K=4, I=128, seed=41)
    write_layer(tmp_path, L, layer=2, n_shards=3)
    st = k3x.Store(str(tmp_path))
    c = cached(k3x, st, L, 2, 12)
    first = [3, 7, 1, 20, 11, 0, 9, 14, 5, 22]
    assert c.cache_getmany(first) == 10
    assert all(c.cache_resident(e) == 1 for e in first)
    assert c.cache_resident(2) == 0
    s = c.cache_stats()
    assert s["misses"] == 10 and s["bytes_read"] == 10 * run_bytes(L) and s["resident"] == 10
    assert c.cache_getmany([3, 7, 1, 20, 11, 16, 17, 18]) == 8
    s = c.cache_stats()
    assert s["misses"] == 13 and s["hits"] == 5 and s["resident"] == 12 and s["evictions"] == 1
    with pytest.raises(k3x.K3XError) as ei:
        c.cache_getmany(list(range(13)))
    assert ei.value.status == -2
    full = bank_layer(k3x, L)
    x = L.x(6, bf16=False, stream_sub=2)
    for t in range(6):
        of, i_f, _ = dev_forward(torch, k3x, full, x[t:t + 1])
        oc, i_c, _ = dev_forward(torch, k3x, c, x[t:t + 1])
        assert np.array_equal(i_f, i_c)
        assert np.array_equal(of.view(np.uint32), oc.view(np.uint32))
    c.close(); full.close(); st.close()


def test_cached_layer_prefill_call(torch, k3x, tmp_path):
    """A 20-token call on a cached layer runs as decode-path calls of 8 tokens: equal bit
    for bit to the resident layer's decode path on the same groups, within the parity
    bar of the oracle."""
    say("case: 20-token call on a cached layer (every expert fits)")
    L = synth.tiny(seed=42)
    write_layer(tmp_path, L, layer=1)
    st = k3x.Store(str(tmp_path))
    c = cached(k3x, st, L, 1, L.E)
    full = bank_layer(k3x, L)
    x = L.x(20, bf16=False, stream_sub=4)
    oc, ic, _ = dev_forward(torch, k3x, c, x)
    of, i_f = decode_chunks(torch, k3x, full, x)
    assert np.array_equal(ic, i_f)
    assert np.array_equal(oc.view(np.uint32), of.view(np.uint32))
    o, oi, _, _ = L.oracle_moe(x)
    assert np.array_equal(ic, oi) and synth.rel_l2(oc, o) < TOL
    c.close(); full.close(); st.close()


@pytest.mark.parametrize("T", [1, 5, 20])
@pytest.mark.parametrize("latent", [False, True])
def test_cache_only_resident_layer(torch, k3x, T, latent):
    """A resident layer with cache-only routing over a given mask (about half the
    experts): against ko_moe_cache_only."""
    say(f"case: cache-only routing, resident layer, half the experts marked, T={T}, latent={latent}")
    L = synth.tiny_latent(seed=3) if latent else synth.tiny(seed=43)
    res = (np.random.default_rng(T).random(L.E) < 0.5).astype(np.int32)
    layer = bank_layer(k3x, L)
    layer.set_cache_only(True, res)
    x = L.x(T, bf16=False, stream_sub=6)
    out, idx, wt = dev_forward(torch, k3x, layer, x)
    o, oi, ow = L.oracle_moe_cache_only(x, res)
    assert np.array_equal(idx, oi)
    np.testing.assert_allclose(wt, ow, rtol=1e-6)
    err = synth.rel_l2(out, o)
    say(f"  rel_l2 vs the oracle {err:.3e}")
    assert err < TOL
    layer.set_cache_only(False)
    out2, idx2, _ = dev_forward(torch, k3x, layer, x)
    e, ei, _, _ = L.oracle_moe(x)
    assert np.array_equal(idx2, ei) and synth.rel_l2(out2, e) < TOL
    layer.close()


def test_cache_only_no_resident_expert(torch, k3x):
    """Nothing resident: every token's routed part is empty, the output is the shared
    expert's (plus the residual)."""
    say("case: cache-only routing with no resident expert")
    L = synth.tiny(seed=44)
    layer = bank_layer(k3x, L)
    res = np.zeros(L.E, np.int32)
    layer.set_cache_only(True, res)
    x = L.x(3, bf16=False)
    out, idx, _ = dev_forward(torch, k3x, layer, x)
    o, oi, _ = L.oracle_moe_cache_only(x, res)
    assert np.array_equal(idx, oi)
    assert synth.rel_l2(out, o) < TOL
    layer.close()


def test_cache_only_cached_layer_reads_nothing(torch, k3x, tmp_path):
    """A cached layer with cache-only routing over its own HBM residency: after warming
    some experts, draft tokens route among them only and read no expert from the store;
    against the oracle over the residency at the time."""
    say("case: cache-only routing over a cached layer's HBM residency")
    L = synth.tiny(seed=45)
    write_layer(tmp_path, L, layer=0)
    st = k3x.Store(str(tmp_path))
    c = cached(k3x, st, L, 0, 10)
    warm = [0, 2, 3, 5, 8, 9, 12, 15]
    assert c.cache_getmany(warm) == len(warm)
    before = c.cache_stats()
    c.set_cache_only(True)
    x = L.x(12, bf16=False, stream_sub=8)
    out, idx, _ = dev_forward(torch, k3x, c, x)
    after = c.cache_stats()
    assert after["misses"] == before["misses"] and after["bytes_read"] == before["bytes_read"]
    res = np.array([c.cache_resident(e) for e in range(L.E)], np.int32)
    o, oi, _ = L.oracle_moe_cache_only(x, res)
    assert np.array_equal(idx, oi)
    assert synth.rel_l2(out, o) < TOL
    c.close(); st.close()


def test_cached_layer_over_a_supplier(torch, k3x):
    """A cache whose misses come through get() (k3x_moe_layer_create_cached_src), the
    getmany() of each batch of misses called first: equal bit for bit to the resident
    layer, the getmany calls naming exactly the misses; a failing get() is a drop
    (K3X_E_DROP, counted) and the layer keeps working."""
    say("case: expert cache over a get()/getmany() supplier, 7 slots")
    L = synth.tiny(seed=46)
    cfg = layer_cfg(k3x, L)
    asked, fail = [], set()

    def get(lay, e):
        return None if e in fail else L.expert(e)

    def getmany(lay, ex):
        asked.append(list(ex))
        return len(ex)

    c = k3x.MoELayer.from_source_cached(cfg, L.gate, L.bias, get, cfg.topk + 3, L.sh1, L.sh3,
                                        L.sh2, getmany=getmany)
    full = bank_layer(k3x, L)
    x = L.x(10, bf16=False, stream_sub=9)
    for t in range(10):
        of, i_f, _ = dev_forward(torch, k3x, full, x[t:t + 1])
        oc, i_c, _ = dev_forward(torch, k3x, c, x[t:t + 1])
        assert np.array_equal(i_f, i_c)
        assert np.array_equal(of.view(np.uint32), oc.view(np.uint32))
    s = c.cache_stats()
    assert sum(len(a) for a in asked) == s["misses"] and s["evictions"] > 0
    _, inext, _, _ = L.oracle_moe(x[:1])
    victim = next(e for e in inext[0] if not c.cache_resident(int(e)))
    fail.add(int(victim))
    d0 = k3x.expert_drops()
    with pytest.raises(k3x.K3XError) as ei:
        dev_forward(torch, k3x, c, x[:1])
    assert ei.value.status == -5 and k3x.expert_drops() == d0 + 1
    fail.clear()
    oc, _, _ = dev_forward(torch, k3x, c, x[:1])
    of, _, _ = dev_forward(torch, k3x, full, x[:1])
    assert np.array_equal(oc.view(np.uint32), of.view(np.uint32))
    assert k3x.cache_slots_fit(cfg) > 0
    c.close(); full.close()


def test_cache_only_forward_refuses_capture(torch, k3x):
    """A decode call that must read the selection back to the host (cache-only routing,
    or an expert cache) returns K3X_E_ARG on a stream under capture, enqueuing nothing;
    the layer then runs eagerly as before."""
    say("case: cache-only decode call under graph capture is refused")
    L = synth.tiny(seed=44)
    res = (np.random.default_rng(5).random(L.E) < 0.5).astype(np.int32)
    layer = bank_layer(k3x, L)
    layer.set_cache_only(True, res)
    x = L.x(2, bf16=False, stream_sub=8)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g, stream=s):
        try:
            layer.forward(out.data_ptr(), xd.data_ptr(), 2, k3x.K3X_F32, 0, 0, 0, s.cuda_stream)
        except k3x.K3XError as e:
            err = e
    torch.cuda.synchronize()
    assert err is not None and err.status == -1, err            # K3X_E_ARG
    got, idx, wt = dev_forward(torch, k3x, layer, x)
    o, oi, ow = L.oracle_moe_cache_only(x, res)
    assert np.array_equal(idx, oi) and synth.rel_l2(got, o) < TOL
    layer.close()
