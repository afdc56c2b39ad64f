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
