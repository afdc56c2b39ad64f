"""The checkpoint reader (include/k3x_store.h) on the CPU: safetensors shards written
here, indexed and read back through the C ABI (no device calls).

Checks: every tensor's dtype, shape, offset and size against what was written; raw reads;
an expert's six tensors resolved as one contiguous run (the released checkpoint's layout,
k3_load.h:3-22) or scattered (six reads into the canonical layout); the reference's
validation failures (k3_load.c:15-105); malformed files; files written by the
`safetensors` library; and real checkpoint bytes (the reference's fixture mxfp4.json,
layer 1 expert 0 w1, rows 0..63) read back through an expert run and dequantised by the
oracle to the fixture's floats.
"""
import ctypes as C
import os
import struct

import numpy as np
import pytest

from store_util import expert_name, expert_tensors, run_bytes, write_shard

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def small_expert(rng, I=64, X=128):
    return {"p1": rng.integers(0, 256, (I, X // 2), dtype=np.uint8),
            "s1": rng.integers(118, 130, (I, X // 32), dtype=np.uint8),
            "p3": rng.integers(0, 256, (I, X // 2), dtype=np.uint8),
            "s3": rng.integers(118, 130, (I, X // 32), dtype=np.uint8),
            "p2": rng.integers(0, 256, (X, I // 2), dtype=np.uint8),
            "s2": rng.integers(118, 130, (X, I // 32), dtype=np.uint8)}


@pytest.fixture()
def shards(tmp_path):
    """Two shards: layer 1 experts 0..2 (contiguous runs) with a bf16 and an fp32 trunk
    tensor in shard B, layer 2 expert 0 scattered among other tensors in shard A."""
    rng = np.random.default_rng(1)
    ex = {(1, e): small_expert(rng) for e in range(3)}
    ex[(2, 0)] = small_expert(rng)
    trunk_bf16 = rng.integers(0, 65536, (32, 16), dtype=np.uint16)
    trunk_f32 = rng.standard_normal((8, 4)).astype(np.float32)
    b_tensors = [("model.norm.weight", "F32", trunk_f32.shape, trunk_f32.tobytes())]
    for e in range(3):
        b_tensors += expert_tensors(1, e, ex[(1, e)])
    b_tensors.append(("model.embed.weight", "BF16", trunk_bf16.shape, trunk_bf16.tobytes()))
    six = expert_tensors(2, 0, ex[(2, 0)])
    f16 = rng.standard_normal(6).astype(np.float16)
    a_tensors = [six[0], ("pad.one", "F16", f16.shape, f16.tobytes()), six[3], six[1],
                 six[5], six[2], six[4]]
    wa = write_shard(tmp_path / "model-00001-of-00002.safetensors", a_tensors,
                     metadata={"format": "pt"}, pad=5)
    wb = write_shard(tmp_path / "model-00002-of-00002.safetensors", b_tensors)
    (tmp_path / "README.txt").write_text("not a shard")
    written = {}
    for shard, (w, ts) in enumerate(((wa, a_tensors), (wb, b_tensors))):
        for name, dt, shape, raw in ts:
            written[name] = (shard, dt, tuple(shape), w[name][0], len(raw), raw)
    return tmp_path, ex, written


DT = {"U8": 1, "BF16": 2, "F16": 3, "F32": 4}


def test_index_matches_what_was_written(k3x, shards):
    path, ex, written = shards
    st = k3x.Store(str(path))
    assert st.shards() == 2 and st.count() == len(written)
    for name, (shard, dt, shape, off, nb, raw) in written.items():
        t = st.find(name)
        assert t is not None, name
        assert (t.shard, t.dtype, t.ndim) == (shard, DT[dt], len(shape))
        assert tuple(t.shape[:t.ndim]) == shape
        assert (t.off, t.nbytes) == (off, nb)
        assert st.read(name).tobytes() == raw
    assert st.find("model.missing") is None
    st.close()


def test_expert_contiguous_run(k3x, shards):
    path, ex, written = shards
    st = k3x.Store(str(path))
    for e in range(3):
        r, buf = st.expert_load(1, e)
        assert r.contiguous == 1 and r.shard == 1
        assert r.off == written[expert_name(1, e, 1, "weight_packed")][3]
        assert buf.tobytes() == run_bytes(ex[(1, e)])
        d = ex[(1, e)]
        for i, (pk, sk) in enumerate((("p1", "s1"), ("p2", "s2"), ("p3", "s3"))):
            m = r.m[i]
            assert (m.rows, m.pcols, m.scols) == (d[pk].shape[0], d[pk].shape[1], d[sk].shape[1])
            assert buf[m.p_off:m.p_off + m.p_bytes].tobytes() == d[pk].tobytes()
            assert buf[m.s_off:m.s_off + m.s_bytes].tobytes() == d[sk].tobytes()
    st.close()


def test_expert_scattered_run(k3x, shards):
    """Tensors out of order with another tensor between them: six reads into the
    canonical layout, the same bytes."""
    path, ex, written = shards
    st = k3x.Store(str(path))
    r, buf = st.expert_load(2, 0)
    assert r.contiguous == 0 and r.shard == 0
    assert buf.tobytes() == run_bytes(ex[(2, 0)])
    st.close()


def test_supplier_get(k3x, shards):
    """The K3ExpertSrc seam: get() points p1/s1 at w1 (gate), p3/s3 at w3 (up), p2/s2 at w2."""
    path, ex, written = shards
    st = k3x.Store(str(path))
    h = C.c_void_p()
    assert k3x.lib().k3x_store_src_create(st.h, C.byref(h)) == 0
    src = C.cast(h, C.POINTER(k3x.ExpertSrc))
    q = k3x.ExpertQ()
    for e in (2, 0):
        assert src.contents.get(src, 1, e, C.byref(q)) == 0
        d = ex[(1, e)]
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            got = np.ctypeslib.as_array(C.cast(getattr(q, k), C.POINTER(C.c_uint8)),
                                        shape=(d[k].size,))
            assert got.tobytes() == d[k].tobytes(), (e, k)
    assert src.contents.get(src, 1, 7, C.byref(q)) != 0           # absent expert
    assert k3x.lib().k3x_store_src_fetches(h) == 2
    # getmany only advises read-ahead: nothing is made resident (0), get() still reads;
    # an absent expert is an error
    ids = (C.c_int * 2)(0, 2)
    assert src.contents.getmany(src, 1, ids, 2) == 0
    assert k3x.lib().k3x_store_src_fetches(h) == 2
    bad = (C.c_int * 1)(7)
    assert src.contents.getmany(src, 1, bad, 1) < 0
    k3x.lib().k3x_store_src_destroy(h)
    st.close()


def _one_expert_dir(tmp_path, mutate):
    rng = np.random.default_rng(2)
    ts = expert_tensors(0, 0, small_expert(rng))
    ts = mutate(ts)
    write_shard(tmp_path / "m.safetensors", ts)
    return tmp_path


@pytest.mark.parametrize("what", ["missing", "dtype", "group", "rows", "one_dim"])
def test_expert_validation(k3x, tmp_path, what):
    def mutate(ts):
        if what == "missing":
            return [t for t in ts if not t[0].endswith("w2.weight_scale")]
        out = []
        for name, dt, shape, raw in ts:
            if name.endswith("w3.weight_scale"):
                if what == "dtype":
                    dt, shape, raw = "F16", (shape[0], shape[1] // 2), raw
                elif what == "group":                   # 16-element groups
                    shape, raw = (shape[0], shape[1] * 2), raw + raw
                elif what == "rows":
                    shape, raw = (shape[0] - 1, shape[1]), raw[:(shape[0] - 1) * shape[1]]
                elif what == "one_dim":
                    shape = (shape[0] * shape[1],)
            out.append((name, dt, shape, raw))
        return out
    st = k3x.Store(str(_one_expert_dir(tmp_path, mutate)))
    with pytest.raises(k3x.K3XError):
        st.expert_ref(0, 0)
    st.close()


def test_expert_split_across_shards(k3x, tmp_path):
    rng = np.random.default_rng(3)
    ts = expert_tensors(0, 0, small_expert(rng))
    write_shard(tmp_path / "a.safetensors", ts[:4])
    write_shard(tmp_path / "b.safetensors", ts[4:])
    st = k3x.Store(str(tmp_path))
    with pytest.raises(k3x.K3XError):
        st.expert_ref(0, 0)
    st.close()


@pytest.mark.parametrize("what", ["truncated", "bytes_vs_shape", "bad_json", "hdr_len",
                                  "dup_name", "dtype"])
def test_malformed_shards_rejected(k3x, tmp_path, what):
    x = np.arange(12, dtype=np.float32)
    p = tmp_path / "m.safetensors"
    if what == "dup_name":
        write_shard(p, [("a", "F32", x.shape, x.tobytes())])
        write_shard(tmp_path / "n.safetensors", [("a", "F32", x.shape, x.tobytes())])
    elif what == "dtype":
        write_shard(p, [("a", "F64", (6,), x.tobytes())])
    elif what == "bytes_vs_shape":
        write_shard(p, [("a", "F32", (13,), x.tobytes())])
    else:
        write_shard(p, [("a", "F32", x.shape, x.tobytes())])
        raw = bytearray(p.read_bytes())
        if what == "truncated":
            raw = raw[:-4]
        elif what == "bad_json":
            n = struct.unpack("<Q", raw[:8])[0]
            raw[8 + n - 1:8 + n] = b"]"
        elif what == "hdr_len":
            raw[:8] = struct.pack("<Q", len(raw) + 10)
        p.write_bytes(bytes(raw))
    with pytest.raises(k3x.K3XError):
        k3x.Store(str(tmp_path))


@pytest.mark.parametrize("shape,nbytes", [([2 ** 62 + 1], 4), ([2 ** 61 + 1, 2], 8)])
def test_overflowing_shape_rejected(k3x, tmp_path, shape, nbytes):
    """A header whose element count times 4 wraps around to the tensor's byte count
    (2^64 + nbytes) is rejected, not indexed."""
    raw = np.zeros(nbytes, np.uint8).tobytes()
    write_shard(tmp_path / "m.safetensors", [("a", "F32", tuple(shape), raw)])
    with pytest.raises(k3x.K3XError):
        k3x.Store(str(tmp_path))


def test_huge_offsets_rejected(k3x, tmp_path):
    """data_offsets near 2^63 (their sum with the header length would wrap) are rejected."""
    p = tmp_path / "m.safetensors"
    big = 2 ** 63 - 4
    hdr = ('{"a": {"dtype": "U8", "shape": [4], "data_offsets": [%d, %d]}}' % (big, big + 4)).encode()
    if big + 4 >= 2 ** 63:
        hdr = ('{"a": {"dtype": "U8", "shape": [4], "data_offsets": [%d, %d]}}'
               % (big - 4, big)).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 4)
    with pytest.raises(k3x.K3XError):
        k3x.Store(str(tmp_path))


def test_supplier_refuses_wrong_shaped_expert(k3x, tmp_path):
    """A supplier made for a layer's expert shape fails get() (a drop for the layer) for an
    expert of another shape, instead of pointing the upload at short arrays; the plain
    supplier still refuses an expert whose three matrices disagree."""
    rng = np.random.default_rng(4)
    write_shard(tmp_path / "m.safetensors",
                expert_tensors(0, 0, small_expert(rng, I=64, X=128)) +
                expert_tensors(0, 1, small_expert(rng, I=32, X=128)))
    st = k3x.Store(str(tmp_path))
    q = k3x.ExpertQ()
    h = C.c_void_p()
    assert k3x.lib().k3x_store_src_create_for(st.h, 64, 128, C.byref(h)) == 0
    src = C.cast(h, C.POINTER(k3x.ExpertSrc))
    assert src.contents.get(src, 0, 0, C.byref(q)) == 0
    assert src.contents.get(src, 0, 1, C.byref(q)) != 0        # 32 rows, not 64
    k3x.lib().k3x_store_src_destroy(h)
    assert k3x.lib().k3x_store_src_create(st.h, C.byref(h)) == 0
    src = C.cast(h, C.POINTER(k3x.ExpertSrc))
    assert src.contents.get(src, 0, 1, C.byref(q)) == 0        # consistent on its own
    k3x.lib().k3x_store_src_destroy(h)
    st.close()


def test_empty_directory_rejected(k3x, tmp_path):
    with pytest.raises(k3x.K3XError):
        k3x.Store(str(tmp_path))


def test_reads_files_of_the_safetensors_library(k3x, tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(4)
    d = small_expert(rng)
    tensors = {expert_name(3, 5, m, k): d[key] for m, k, key in
               ((1, "weight_packed", "p1"), (1, "weight_scale", "s1"),
                (2, "weight_packed", "p2"), (2, "weight_scale", "s2"),
                (3, "weight_packed", "p3"), (3, "weight_scale", "s3"))}
    tensors["model.x"] = rng.standard_normal((3, 5)).astype(np.float32)
    save_file(tensors, str(tmp_path / "lib.safetensors"), metadata={"k": "v"})
    st = k3x.Store(str(tmp_path))
    assert st.count() == 7
    assert st.read("model.x").tobytes() == tensors["model.x"].tobytes()
    r, buf = st.expert_load(3, 5)
    assert buf.tobytes() == run_bytes(d)
    st.close()


def test_real_checkpoint_bytes_through_an_expert_run(k3x, tmp_path):
    """The released checkpoint's layer 1 expert 0 w1 (rows 0..63, from the reference's
    fixture) as the first rows of a K3-geometry expert's gate: read back through the
    contiguous run and dequantised by the oracle to the fixture's floats."""
    from oracle_lib import F32P, U8P, oracle, ptr
    g = np.load(os.path.join(GOLD, "ref_mxfp4.npz"))
    I, X = 3072, 3584
    rng = np.random.default_rng(5)
    d = {"p1": rng.integers(0, 256, (I, X // 2), dtype=np.uint8),
         "s1": rng.integers(118, 130, (I, X // 32), dtype=np.uint8),
         "p3": rng.integers(0, 256, (I, X // 2), dtype=np.uint8),
         "s3": rng.integers(118, 130, (I, X // 32), dtype=np.uint8),
         "p2": rng.integers(0, 256, (X, I // 2), dtype=np.uint8),
         "s2": rng.integers(118, 130, (X, I // 32), dtype=np.uint8)}
    d["p1"][:64] = g["packed"]
    d["s1"][:64] = g["scales"]
    write_shard(tmp_path / "k3.safetensors", expert_tensors(1, 0, d))
    st = k3x.Store(str(tmp_path))
    r, buf = st.expert_load(1, 0)
    assert r.contiguous == 1 and r.nbytes == 17547264          # k3_load.h:5-8
    m = r.m[0]
    packed = np.ascontiguousarray(buf[m.p_off:m.p_off + m.p_bytes].reshape(I, X // 2)[:64])
    scales = np.ascontiguousarray(buf[m.s_off:m.s_off + m.s_bytes].reshape(I, X // 32)[:64])
    assert np.array_equal(packed, g["packed"]) and np.array_equal(scales, g["scales"])
    y = np.empty((64, X), np.float32)
    oracle().ko_mxfp4_dequant(ptr(y, F32P), ptr(packed, U8P), ptr(scales, U8P), 64, X // 2, 32)
    assert np.array_equal(y, g["expected"])
    st.close()


@pytest.mark.parametrize("nslot", [0, 4, 17])
def test_cached_layer_slot_bounds(k3x, shards, nslot):
    """k3x_moe_layer_create_cached refuses fewer than topk + 1 slots or more slots than
    experts before it touches a device (k3_cache_init's lower bound)."""
    path, _, _ = shards
    st = k3x.Store(str(path))
    cfg = k3x.make_cfg(256, 16, 4, 128, 1, 1, 2.5)
    gate = np.zeros((16, 256), np.float32)
    with pytest.raises(k3x.K3XError) as ei:
        k3x.MoELayer.from_store_cached(cfg, gate, None, st, 1, nslot)
    assert ei.value.status == -1
    st.close()
