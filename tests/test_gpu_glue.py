"""The decoder-layer glue on the device against the oracle: the block attention-residual
aggregation (k3x_attn_res vs ko_attn_res, which is bitwise the reference's k3_attn_res),
and the MoE half of a decoder layer (k3x_moe_half vs ko_moe_half), eagerly and replayed
from a captured graph."""
import ctypes as C

import numpy as np
import pytest

import synth
from gpu_util import bank_layer, say
from oracle_lib import F32P, oracle, ptr

pytestmark = pytest.mark.gpu


def oracle_attn_res(blocks, nb, pref, fold, eps):
    T, n = pref.shape
    out = np.empty_like(pref)
    for t in range(T):
        src = np.ascontiguousarray(np.concatenate([blocks[t, :nb], pref[t:t + 1]]), np.float32)
        oracle().ko_attn_res(ptr(out[t], F32P), ptr(src, F32P), ptr(fold, F32P), nb + 1, n, eps)
    return out


@pytest.mark.parametrize("n,nb", [(256, 0), (7168, 3), (7168, 8)])
def test_attn_res_vs_oracle(torch, k3x, n, nb):
    say(f"case: attn_res n={n} nb={nb}, 5 rows")
    T, maxb = 5, 9
    rng = np.random.default_rng(n + nb)
    blocks = (rng.standard_normal((T, maxb, n)) * rng.uniform(0.2, 5, (T, maxb, 1))).astype(np.float32)
    pref = rng.standard_normal((T, n)).astype(np.float32)
    fold = (rng.standard_normal(n) * 0.05).astype(np.float32)
    bd, pd, fd = (torch.from_numpy(a).cuda() for a in (blocks, pref, fold))
    hd = torch.empty_like(pd)
    k3x.attn_res(hd.data_ptr(), bd.data_ptr(), maxb, nb, pd.data_ptr(), fd.data_ptr(), n, T, 1e-5,
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got, want = hd.cpu().numpy(), oracle_attn_res(blocks, nb, pref, fold, 1e-5)
    same = float(np.mean(got.view(np.uint32) == want.view(np.uint32)))
    err = synth.rel_l2(got, want)
    say(f"  rel_l2={err:.3e}, bitwise-equal fraction {same:.4f}")
    assert err < 1e-6


@pytest.mark.parametrize("nb", [0, 3])
def test_attn_res_cancelling_keys_bitwise(torch, k3x, nb):
    """Sources whose keys cancel: every source row carries +B and -B at columns p and
    p + 1 where fold holds 2^20 twice, so the normalised pair's products cancel but first
    round away low bits of the partial sum they meet, which depends on the order of the
    additions; with nb = 3, block 0 of each row is instead a row at the RMSNorm scale's
    rounding midpoint (synth.rms_window_row).  The kernel's tree sums cannot prove
    those floats, forms them again as the reference's chains, and the output is the
    reference's bit for bit.  Teeth: a four-chain order changes most keys' floats."""
    say(f"case: attn_res with cancelling keys and RMSNorm window rows, nb={nb}, bitwise")
    T, maxb, n, p, eps = 4, 4, 1024, 512, 1e-5
    rng = np.random.default_rng(90 + nb)
    blocks = rng.standard_normal((T, maxb, n)).astype(np.float32)
    pref = rng.standard_normal((T, n)).astype(np.float32)
    fold = (rng.standard_normal(n) * 0.05).astype(np.float32)
    fold[p] = fold[p + 1] = np.float32(2.0 ** 20)
    for t in range(T):
        for s in range(maxb):
            b = np.float32(2.0 ** 10) * (1 if (t + s) % 2 else -1)
            blocks[t, s, p], blocks[t, s, p + 1] = b, -b
        pref[t, p], pref[t, p + 1] = np.float32(2.0 ** 10), np.float32(-2.0 ** 10)
        if nb > 0:
            blocks[t, 0] = synth.rms_window_row(n, eps, 300 + t)
    # teeth (CPU): keys by the reference's chain against a four-chain order
    chg = 0
    srcs = [blocks[t, s] for t in range(T) for s in range(nb)] + [pref[t] for t in range(T)]
    for v in srcs:
        ss = float(np.sum(v.astype(np.float64) ** 2))
        inv = synth.rms_inv(ss, n, eps)
        term = (v * inv).astype(np.float64) * fold.astype(np.float64)
        seq = 0.0
        ch = [0.0] * 4
        for i in range(n):
            seq += term[i]
            ch[i % 4] += term[i]
        chg += np.float32(seq) != np.float32((ch[0] + ch[1]) + (ch[2] + ch[3]))
    say(f"  keys that a four-chain order changes: {chg} of {len(srcs)}")
    assert chg >= len(srcs) // 3
    bd, pd, fd = (torch.from_numpy(a).cuda() for a in (blocks, pref, fold))
    hd = torch.empty_like(pd)
    k3x.attn_res(hd.data_ptr(), bd.data_ptr(), maxb, nb, pd.data_ptr(), fd.data_ptr(), n, T, eps,
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got, want = hd.cpu().numpy(), oracle_attn_res(blocks, nb, pref, fold, eps)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def oracle_half(L, h, pref, blocks, nb, fold, post, eps):
    cfg = L.ko_cfg()
    w, cb, keep = L._weights()
    T, H = pref.shape
    h = h.copy(); p = pref.copy()
    b = np.ascontiguousarray(blocks, np.float32)
    oracle().ko_moe_half(ptr(h, F32P), ptr(p, F32P), ptr(b, F32P), b.shape[1], nb,
                         ptr(fold, F32P), ptr(post, F32P), eps, T, C.byref(cfg), C.byref(w))
    return h, p


def half_inputs(L, T, maxb, seed):
    rng = np.random.default_rng(seed)
    H = L.H
    blocks = (rng.standard_normal((T, maxb, H)) * 0.5).astype(np.float32)
    pref = L.x(T, bf16=False, stream_sub=seed)
    fold = (rng.standard_normal(H) * 0.05).astype(np.float32)
    post = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    return blocks, pref, fold, post


@pytest.mark.parametrize("latent,T", [(False, 1), (False, 12), (True, 4)])
def test_moe_half_vs_oracle(torch, k3x, latent, T):
    say(f"case: MoE half of a decoder layer, latent={latent}, T={T}, 3 block residuals")
    L = synth.tiny_latent(seed=33) if latent else synth.tiny(seed=33)
    layer = bank_layer(k3x, L)
    nb, maxb = 3, 4
    blocks, pref, fold, post = half_inputs(L, T, maxb, 7 + T)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in
         (("b", blocks), ("p", pref), ("f", fold), ("n", post))}
    h = torch.empty_like(d["p"]); hin = torch.empty_like(d["p"])
    layer.moe_half(h.data_ptr(), d["p"].data_ptr(), d["b"].data_ptr(), maxb, nb,
                   d["f"].data_ptr(), d["n"].data_ptr(), 1e-5, T, hin.data_ptr(),
                   torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    layer.check()
    wh, wp = oracle_half(L, np.zeros_like(pref), pref, blocks, nb, fold, post, 1e-5)
    eh, ep = synth.rel_l2(h.cpu().numpy(), wh), synth.rel_l2(d["p"].cpu().numpy(), wp)
    say(f"  rel_l2 h={eh:.3e} pref={ep:.3e}")
    assert eh < 1e-3 and ep < 1e-3
    assert torch.equal(h, d["p"])
    layer.close()


def test_moe_half_graph_replays(torch, k3x):
    """One layer's glue + MoE captured once, replayed on new inputs with eager work and
    synchronisations between the replays; every replay equals the eager result."""
    say("case: MoE half captured in a graph, 4 replays with eager copies between")
    L = synth.tiny(seed=34)
    layer = bank_layer(k3x, L)
    T, nb, maxb = 2, 2, 2
    H = L.H
    bd = torch.empty((T, maxb, H), dtype=torch.float32, device="cuda")
    pd = torch.empty((T, H), dtype=torch.float32, device="cuda")
    fd = torch.empty((H,), dtype=torch.float32, device="cuda")
    nd = torch.empty((H,), dtype=torch.float32, device="cuda")
    h = torch.empty_like(pd); hin = torch.empty_like(pd)
    s = torch.cuda.Stream()

    def load(seed):
        blocks, pref, fold, post = half_inputs(L, T, maxb, seed)
        bd.copy_(torch.from_numpy(blocks)); pd.copy_(torch.from_numpy(pref))
        fd.copy_(torch.from_numpy(fold)); nd.copy_(torch.from_numpy(post))

    def run(stream):
        layer.moe_half(h.data_ptr(), pd.data_ptr(), bd.data_ptr(), maxb, nb, fd.data_ptr(),
                       nd.data_ptr(), 1e-5, T, hin.data_ptr(), stream)

    load(100)
    with torch.cuda.stream(s):
        run(s.cuda_stream)                      # eager warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(s.cuda_stream)
    torch.cuda.synchronize()
    for r in range(4):
        load(200 + r)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_h, got_p = h.clone(), pd.clone()
        load(200 + r)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            run(s.cuda_stream)
        torch.cuda.synchronize()
        say(f"  replay {r}")
        assert torch.equal(got_h, h) and torch.equal(got_p, pd)
    layer.check()
    layer.close()


def oracle_half_v(L, pref, blocks, nbv, nbs, fold, post, eps=1e-5):
    from oracle_lib import I32P
    cfg = L.ko_cfg()
    w, cb, keep = L._weights()
    T = pref.shape[0]
    h = np.zeros_like(pref); p = pref.copy()
    b = np.ascontiguousarray(blocks, np.float32)
    nbv = np.ascontiguousarray(nbv, np.int32)
    oracle().ko_moe_half_v(ptr(h, F32P), ptr(p, F32P), ptr(b, F32P), b.shape[1], ptr(nbv, I32P),
                           nbs, ptr(fold, F32P), ptr(post, F32P), eps, T, C.byref(cfg),
                           C.byref(w))
    return h, p


def test_attn_res_v_per_row_counts(torch, k3x):
    """Block counts read per row from a device array (k3_ops.c:2481-2493, nbs 1): each row
    against the oracle with its own count; a count past maxb gives a NaN row; nbs 0 is
    one count for every row."""
    n, T, maxb = 7168, 6, 5
    say(f"case: attn_res_v n={n}, {T} rows, per-row counts")
    rng = np.random.default_rng(11)
    blocks = (rng.standard_normal((T, maxb, n)) * rng.uniform(0.2, 5, (T, maxb, 1))).astype(np.float32)
    pref = rng.standard_normal((T, n)).astype(np.float32)
    fold = (rng.standard_normal(n) * 0.05).astype(np.float32)
    bd, pd, fd = (torch.from_numpy(a).cuda() for a in (blocks, pref, fold))
    hd = torch.empty_like(pd)
    st = torch.cuda.current_stream().cuda_stream
    counts = [3, 0, 5, 1, 4, 2]
    nbd = torch.tensor(counts, dtype=torch.int32, device="cuda")
    k3x.attn_res_v(hd.data_ptr(), bd.data_ptr(), maxb, nbd.data_ptr(), 1, pd.data_ptr(),
                   fd.data_ptr(), n, T, 1e-5, st)
    torch.cuda.synchronize()
    got = hd.cpu().numpy()
    for t, nb in enumerate(counts):
        want = oracle_attn_res(blocks[t:t + 1], nb, pref[t:t + 1], fold, 1e-5)[0]
        err = synth.rel_l2(got[t], want)
        say(f"  row {t} nb={nb}: rel_l2={err:.3e}")
        assert err < 1e-6
    # one shared count (nbs 0) equals the host-count entry point bit for bit
    k3x.attn_res_v(hd.data_ptr(), bd.data_ptr(), maxb, nbd.data_ptr() + 4 * 4, 0, pd.data_ptr(),
                   fd.data_ptr(), n, T, 1e-5, st)
    h2 = torch.empty_like(pd)
    k3x.attn_res(h2.data_ptr(), bd.data_ptr(), maxb, 4, pd.data_ptr(), fd.data_ptr(), n, T, 1e-5, st)
    torch.cuda.synchronize()
    assert torch.equal(hd, h2)
    # a count past maxb: that row is NaN, the others are computed
    bad = torch.tensor([1, maxb + 1, 2, -1, 0, 3], dtype=torch.int32, device="cuda")
    k3x.attn_res_v(hd.data_ptr(), bd.data_ptr(), maxb, bad.data_ptr(), 1, pd.data_ptr(),
                   fd.data_ptr(), n, T, 1e-5, st)
    torch.cuda.synchronize()
    g = hd.cpu().numpy()
    assert np.isnan(g[1]).all() and np.isnan(g[3]).all()
    assert np.isfinite(g[[0, 2, 4, 5]]).all()


@pytest.mark.parametrize("latent,T", [(False, 5), (True, 3), (False, 12)])
def test_moe_half_v_vs_oracle(torch, k3x, latent, T):
    """The MoE half with a block count per row, against ko_moe_half_v (itself bitwise the
    reference's functions composed as the decoder layer's MLP half)."""
    say(f"case: MoE half with per-row counts, latent={latent}, T={T}")
    L = synth.tiny_latent(seed=35) if latent else synth.tiny(seed=35)
    layer = bank_layer(k3x, L)
    maxb = 4
    counts = [(3 * t + 1) % (maxb + 1) for t in range(T)]
    blocks, pref, fold, post = half_inputs(L, T, maxb, 21 + T)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in
         (("b", blocks), ("p", pref), ("f", fold), ("n", post))}
    nbd = torch.tensor(counts, dtype=torch.int32, device="cuda")
    h = torch.empty_like(d["p"]); hin = torch.empty_like(d["p"])
    layer.moe_half_v(h.data_ptr(), d["p"].data_ptr(), d["b"].data_ptr(), maxb, nbd.data_ptr(), 1,
                     d["f"].data_ptr(), d["n"].data_ptr(), 1e-5, T, hin.data_ptr(),
                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    layer.check()
    wh, wp = oracle_half_v(L, pref, blocks, counts, 1, fold, post)
    eh, ep = synth.rel_l2(h.cpu().numpy(), wh), synth.rel_l2(d["p"].cpu().numpy(), wp)
    say(f"  counts {counts}: rel_l2 h={eh:.3e} pref={ep:.3e}")
    assert eh < 1e-3 and ep < 1e-3
    assert torch.equal(h, d["p"])
    layer.close()


def test_moe_half_v_graph_replays(torch, k3x):
    """The per-row form captured once; each replay runs with counts and inputs changed on
    the device in between (the counts are read when the graph runs), and equals the eager
    call on the same counts and inputs."""
    say("case: MoE half with per-row counts captured in a graph, 4 replays, counts changed")
    L = synth.tiny(seed=36)
    layer = bank_layer(k3x, L)
    T, maxb = 3, 3
    H = L.H
    bd = torch.empty((T, maxb, H), dtype=torch.float32, device="cuda")
    pd = torch.empty((T, H), dtype=torch.float32, device="cuda")
    fd = torch.empty((H,), dtype=torch.float32, device="cuda")
    nd = torch.empty((H,), dtype=torch.float32, device="cuda")
    nbd = torch.zeros((T,), dtype=torch.int32, device="cuda")
    h = torch.empty_like(pd); hin = torch.empty_like(pd)
    s = torch.cuda.Stream()

    def load(seed, counts):
        blocks, pref, fold, post = half_inputs(L, T, maxb, seed)
        bd.copy_(torch.from_numpy(blocks)); pd.copy_(torch.from_numpy(pref))
        fd.copy_(torch.from_numpy(fold)); nd.copy_(torch.from_numpy(post))
        nbd.copy_(torch.tensor(counts, dtype=torch.int32))
        return blocks, pref, fold, post

    def run(stream):
        layer.moe_half_v(h.data_ptr(), pd.data_ptr(), bd.data_ptr(), maxb, nbd.data_ptr(), 1,
                         fd.data_ptr(), nd.data_ptr(), 1e-5, T, hin.data_ptr(), stream)

    load(300, [1, 2, 0])
    with torch.cuda.stream(s):
        run(s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(s.cuda_stream)
    torch.cuda.synchronize()
    for r, counts in enumerate(([0, 3, 1], [2, 2, 2], [3, 0, 2], [1, 1, 3])):
        blocks, pref, fold, post = load(400 + r, counts)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_h, got_p = h.clone(), pd.clone()
        load(400 + r, counts)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            run(s.cuda_stream)
        torch.cuda.synchronize()
        wh, _ = oracle_half_v(L, pref, blocks, counts, 1, fold, post)
        err = synth.rel_l2(got_h.cpu().numpy(), wh)
        say(f"  replay {r} counts {counts}: rel_l2 vs oracle {err:.3e}")
        assert torch.equal(got_h, h) and torch.equal(got_p, pd)
        assert err < 1e-3
    layer.check()
    layer.close()
