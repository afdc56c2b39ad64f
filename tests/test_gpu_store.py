"""A layer whose routed experts stream from safetensors shards into HBM
(k3x_moe_layer_create_from_store), against the same layer uploaded from a bank: the
re-laid-out experts read back byte for byte and the forward outputs are bitwise equal."""
import numpy as np
import pytest

import synth
from gpu_util import bank_layer, dev_forward, layer_cfg, say
from store_util import expert_tensors, write_shard

pytestmark = pytest.mark.gpu


def write_layer(tmp_path, L, layer, n_shards=2, skip=None):
    per = (L.E + n_shards - 1) // n_shards
    for sh in range(n_shards):
        ts = []
        for e in range(sh * per, min(L.E, (sh + 1) * per)):
            if e != skip:
                ts += expert_tensors(layer, e, L.expert(e))
        write_shard(tmp_path / f"model-{sh:05d}.safetensors", ts)


@pytest.mark.parametrize("latent", [False, True])
def test_layer_from_store_equals_bank(torch, k3x, tmp_path, latent):
    say(f"case: layer streamed from shards (latent={latent}) vs bank upload")
    L = synth.tiny_latent(seed=21) if latent else synth.tiny(seed=21)
    write_layer(tmp_path, L, layer=4)
    st = k3x.Store(str(tmp_path))
    a = k3x.MoELayer.from_store(layer_cfg(k3x, L), L.gate, L.bias, st, 4, L.sh1, L.sh3, L.sh2,
                                down=L.down, up=L.up, latent_norm=L.lnorm)
    b = bank_layer(k3x, L)
    for e in (0, 5, L.E - 1):
        da, db = a.read_expert(e), b.read_expert(e)
        for k in da:
            assert np.array_equal(da[k], db[k]), (e, k)
            assert np.array_equal(da[k], L.expert(e)[k]), (e, k)
    x = L.x(6, bf16=False)
    oa, ia, _ = dev_forward(torch, k3x, a, x)
    ob, ib, _ = dev_forward(torch, k3x, b, x)
    assert np.array_equal(ia, ib)
    assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
    o, idx, _, _ = L.oracle_moe(x)
    assert synth.rel_l2(oa, o) < 1e-3
    a.close(); b.close(); st.close()


def test_missing_expert_is_a_drop(torch, k3x, tmp_path):
    say("case: a shard set missing one expert: K3X_E_DROP, counted")
    L = synth.tiny(seed=22)
    write_layer(tmp_path, L, layer=0, skip=9)
    st = k3x.Store(str(tmp_path))
    d0 = k3x.expert_drops()
    with pytest.raises(k3x.K3XError) as ei:
        k3x.MoELayer.from_store(layer_cfg(k3x, L), L.gate, L.bias, st, 0, L.sh1, L.sh3, L.sh2)
    assert ei.value.status == -5
    assert k3x.expert_drops() == d0 + 1
    st.close()


def run_bytes(L):
    return 3 * (L.I * L.XL // 2 + L.I * L.XL // 32)


@pytest.mark.parametrize("latent", [False, True])
def test_cached_layer_equals_resident(torch, k3x, tmp_path, latent):
    """A layer with an HBM expert cache of topk + 2 slots over the shards, token by token and
    in T = 2 calls, against the same layer with every expert resident: identical indices and
    bitwise equal outputs; the counters add up (hits + misses = experts named, bytes read =
    misses x run, evictions = misses - resident)."""
    say(f"case: expert cache of topk+2 slots (latent={latent}) vs every expert resident")
    L = synth.tiny_latent(seed=23) if latent else synth.tiny(seed=23)
    write_layer(tmp_path, L, layer=3)
    st = k3x.Store(str(tmp_path))
    cfg = layer_cfg(k3x, L)
    kw = dict(down=L.down, up=L.up, latent_norm=L.lnorm)
    full = k3x.MoELayer.from_store(cfg, L.gate, L.bias, st, 3, L.sh1, L.sh3, L.sh2, **kw)
    nslot = cfg.topk + 2
    cache = k3x.MoELayer.from_store_cached(cfg, L.gate, L.bias, st, 3, nslot, L.sh1, L.sh3,
                                           L.sh2, **kw)
    x = L.x(12, bf16=False, stream_sub=3)
    named, seen = 0, set()
    for t in range(12):
        of, i_f, _ = dev_forward(torch, k3x, full, x[t:t + 1])
        oc, i_c, _ = dev_forward(torch, k3x, cache, x[t:t + 1])
        assert np.array_equal(i_f, i_c), t
        assert np.array_equal(of.view(np.uint32), oc.view(np.uint32)), t
        named += len(np.unique(i_c))
        seen |= set(np.unique(i_c).tolist())
    for t in range(0, 6, 2):
        of, i_f, _ = dev_forward(torch, k3x, full, x[t:t + 2])
        if len(np.unique(i_f)) > nslot:
            continue
        oc, i_c, _ = dev_forward(torch, k3x, cache, x[t:t + 2])
        assert np.array_equal(i_f, i_c)
        assert np.array_equal(of.view(np.uint32), oc.view(np.uint32))
        named += len(np.unique(i_c))
    s = cache.cache_stats()
    say(f"  stats {s}, distinct experts {len(seen)}")
    assert s["nslot"] == nslot
    assert s["hits"] + s["misses"] == named
    assert s["bytes_read"] == s["misses"] * run_bytes(L)
    assert s["resident"] == min(nslot, s["misses"])
    assert s["evictions"] == s["misses"] - s["resident"]
    assert s["misses"] >= len(seen) and s["evictions"] > 0
    o, _, _, _ = L.oracle_moe(x[:1])
    of, _, _ = dev_forward(torch, k3x, cache, x[:1])
    assert synth.rel_l2(of, o) < 1e-3
    cache.close(); full.close(); st.close()


def test_cache_pin_prefill_and_capacity(torch, k3x, tmp_path):
    """A pinned expert stays resident through later tokens; a call naming more experts
    than slots returns K3X_E_SHAPE (a 16-token call runs as 8-token decode calls, whose
    first group names more than topk + 1) and the layer keeps working."""
    say("case: expert cache pinning, prefill refusal, capacity")
    L = synth.tiny(seed=24)
    write_layer(tmp_path, L, layer=0)
    st = k3x.Store(str(tmp_path))
    cfg = layer_cfg(k3x, L)
    cache = k3x.MoELayer.from_store_cached(cfg, L.gate, L.bias, st, 0, cfg.topk + 1, L.sh1,
                                           L.sh3, L.sh2)
    cache.cache_pin(7)
    x = L.x(16, bf16=False, stream_sub=5)
    for t in range(8):
        dev_forward(torch, k3x, cache, x[t:t + 1])
    assert np.array_equal(cache.read_expert(7)["p1"], L.expert(7)["p1"])
    _, idx8, _, _ = L.oracle_moe(x[:8])
    with pytest.raises(k3x.K3XError) as ei:
        dev_forward(torch, k3x, cache, x)                 # T = 16: groups of 8 tokens
    assert ei.value.status == -2
    assert len(np.unique(idx8)) > cfg.topk + 1
    with pytest.raises(k3x.K3XError) as ei:
        dev_forward(torch, k3x, cache, x[:8])             # more experts than slots
    assert ei.value.status == -2
    o, _, _, _ = L.oracle_moe(x[:1])
    of, _, _ = dev_forward(torch, k3x, cache, x[:1])
    assert synth.rel_l2(of, o) < 1e-3
    cache.cache_pin(7, False)
    cache.close(); st.close()
