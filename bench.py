"""Benchmark of the MoE block on one MI355X.

Default workload: the full-size K2-class MoE layer (hidden 7168, 384 routed experts
top-8, expert intermediate 2048 in MXFP4 = E2M1 codes + E8M0 per-32 scales, one bf16
shared expert of intermediate 2048, sigmoid router with bias, routed scale 2.5) decoding
batch-1 tokens.  A step is one layer invocation on one token; the tokens rotate over a
pool of 64 distinct seeded bf16 N(0,1) activations resident in HBM, and the steps rotate
over 4 layers of that shape, so every step reads its weights from HBM (a single layer
called back to back finds its router and shared expert, 99 MB, still in the 256 MB
last-level cache; that figure is reported as warm_one_layer_us_per_token).  Weights are
synthetic (seeded generator, random init).  The record also carries the T=8 verify leg,
the 2048-token prefill leg, the 8-layer stack leg, the K3 LatentMoE decode leg and a
trunk-product leg.

Prints ONE JSON line (rank 0):
  value        microseconds per token for the whole layer (lower is better)
  roofline     the dominant kernel's algorithmic HBM bytes per launch over its average
               duration (HIP events on the launch stream), against 8 TB/s
  cpu_baseline the reference's own C kernels composing the same layer on this host's
               cores (oracle/_ref, "reference"), or the oracle port when that library is
               absent ("port"), on a bounded sample of tokens
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "kimi-k3-for-me_amd")

H, E, K, I, SI = 7168, 384, 8, 2048, 2048
HBM_PEAK_GBS = 8000.0
B_EXPERT = 3 * I * H // 2 + 3 * I * H // 32          # 23,396,352 bytes per routed expert
B_SHARED = 3 * SI * H * 2                             # 88,080,384
B_ROUTER = E * H * 4 + E * 4                          # 11,011,584
NROT = 4                                              # layers the decode steps rotate over


def load_k3x():
    spec = importlib.util.spec_from_file_location("k3x", os.path.join(PKG, "k3x.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


KERNELS = ["k1_router_bset", "k2_gateup", "k3_down"]


def kernel_bytes(U, T):
    """Algorithmic HBM bytes per launch of the three decode kernels (each weight byte
    once; activations included): k1 the router weights, k2 the scores, the shared expert's and the
    unique experts' gate/up weights, k3 the unique experts' and the shared expert's down
    weights and the output."""
    k1 = B_ROUTER + T * H * 2
    k2 = 2 * SI * H * 2 + U * 2 * (I * H // 2 + I * H // 32) + 2 * T * E * 4
    k3 = U * (H * I // 2 + H * I // 32) + H * SI * 2 + T * H * 4
    return dict(zip(KERNELS, (k1, k2, k3)))


PREFILL_T = 2048


def prefill_leg(torch, k3x, reps=5):
    """Prefill of one 2048-token chunk of bf16 N(0,1) activations through the full-size
    layer with Zipf-skewed routing (bias alpha*(pi(e)+1)^-1.1, alpha 1.0, seeded
    permutation pi).  Algorithmic bytes: every weight byte of the experts the chunk uses,
    the shared expert and the router, once, plus the activations in and out.  FLOPs: 2 per
    multiply-add of the routed experts (T*K*3*I*H), the shared expert and the router."""
    T = PREFILL_T
    cfg = k3x.make_cfg(H, E, K, I, 1, 1, 2.5)
    layer = k3x.MoELayer.synthetic(cfg, seed=3, zipf_alpha=1.0)
    xs = k3x.synth_normal_f32(T * H, k3x.synth_key(3, 0, k3x.STREAM_X, 5))
    x = torch.from_numpy(xs.reshape(T, H)).cuda().to(torch.bfloat16).contiguous()
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((T, K), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream

    def run():
        layer.forward(out.data_ptr(), x.data_ptr(), T, k3x.K3X_BF16, 0, idx.data_ptr(),
                      wt.data_ptr(), stream=sh)

    def timed():
        with torch.cuda.stream(stream):
            run()
            run()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                run()
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def rates(ms):
        used = int(torch.unique(idx).numel())
        layer_bytes = used * B_EXPERT + B_SHARED + B_ROUTER + T * H * 2 + T * H * 4
        flops = 2.0 * T * (K * 3 * I * H + 3 * I * H + E * H)
        return {"tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_chunk": round(ms, 3),
                "experts_used": used,
                "hbm_gbs": round(layer_bytes / (ms * 1e-3) / 1e9, 1),
                "hbm_frac": round(layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                "mfma_frac_mxfp4_peak": round(flops / (ms * 1e-3) / 1e12 / 10100.0, 4),
                "mfma_frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / 2500.0, 4)}

    ms = timed()
    rec = {"workload": f"prefill {T} bf16 tokens, Zipf-skewed routing (alpha 1.0, s 1.1)"}
    rec.update(rates(ms))
    rec["reps"] = reps
    # the opt-in MXFP8-activation mode on the same layer and input: scaled matrix cores
    # for the routed products; its distance from the exact mode is reported beside it
    exact_out, exact_idx = out.clone(), idx.clone()
    layer.set_prefill_mode(k3x.K3X_PREFILL_MXFP8)
    ms_mx = timed()
    mx = {"mode": "K3X_PREFILL_MXFP8 (opt-in): routed products on v_mfma_scale_f32_32x32x64_f8f6f4, "
                  "activations quantised to MXFP8"}
    mx.update(rates(ms_mx))
    d = (out.double() - exact_out.double()).norm() / exact_out.double().norm()
    mx["rel_l2_vs_exact_mode"] = float(f"{float(d):.3e}")
    mx["same_experts_as_exact_mode"] = bool(torch.equal(idx, exact_idx))
    rec["mxfp8"] = mx
    layer.close()
    del x, out, idx, wt, exact_out, exact_idx
    torch.cuda.empty_cache()
    return rec


STACK_LAYERS, STACK_TOKENS = 8, 256


def stack_leg(torch, k3x):
    """Eight stacked full-size layers (seed 10+l each, about 73 GB resident), each step
    h = h + MoE_l(RMSNorm_l(h)) with norm weights 1 + N(0, 0.1), replayed from one HIP
    graph per token; 256 consecutive batch-1 tokens from a seeded N(0,1) stream.  The
    token copies in and out stay on the stream between replays."""
    cfg = k3x.make_cfg(H, E, K, I, 1, 1, 2.5)
    layers, norms = [], []
    for l in range(STACK_LAYERS):
        layers.append(k3x.MoELayer.synthetic(cfg, seed=10 + l, layer=l))
        w = k3x.synth_normal_f32(H, k3x.synth_key(10 + l, l, k3x.STREAM_NORM, 0), 1.0, 0.1)
        norms.append(torch.from_numpy(w).cuda())
    xs = k3x.synth_normal_f32(STACK_TOKENS * H, k3x.synth_key(10, 0, k3x.STREAM_X, 7))
    x = torch.from_numpy(xs.reshape(STACK_TOKENS, H)).cuda()
    out = torch.empty_like(x)
    h = torch.empty((1, H), dtype=torch.float32, device="cuda")
    S = k3x.Stack(layers, [w.data_ptr() for w in norms], eps=1e-5, max_T=1)
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream

    def step(t):
        h.copy_(x[t:t + 1])
        S.forward(h.data_ptr(), 1, sh)
        out[t:t + 1].copy_(h)

    with torch.cuda.stream(stream):
        for t in range(8):
            step(t)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for t in range(STACK_TOKENS):
            step(t)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    us_tok = ms * 1e3 / STACK_TOKENS
    per_layer_bytes = K * B_EXPERT + B_SHARED + B_ROUTER + H * 4 * 4
    gbs = STACK_LAYERS * per_layer_bytes / (us_tok * 1e-6) / 1e9
    finite = bool(torch.isfinite(out).all().item())
    # tokens 0 and 255 again through the layers one call at a time, outside the graph
    # (k3x_rmsnorm, then the MoE call with the residual): the replayed graph's outputs
    # must equal them bit for bit (the oracle's parity at this width is a GPU test)
    same = True
    with torch.cuda.stream(stream):
        for t in (0, STACK_TOKENS - 1):
            ref = x[t:t + 1].clone()
            y = torch.empty_like(ref)
            for l, w in zip(layers, norms):
                k3x.rmsnorm(y.data_ptr(), ref.data_ptr(), w.data_ptr(), H, 1, 1e-5, sh)
                l.forward(ref.data_ptr(), y.data_ptr(), 1, k3x.K3X_F32, ref.data_ptr(), 0, 0, sh)
            torch.cuda.synchronize()
            same = same and bool(torch.equal(ref, out[t:t + 1]))
    for l in layers:
        l.check()
    S.close()
    for l in layers:
        l.close()
    del x, out, h, norms
    torch.cuda.empty_cache()
    return {"workload": f"{STACK_LAYERS} stacked layers, RMSNorm + MoE + residual each, "
                        f"{STACK_TOKENS} batch-1 tokens, one HIP graph replay per token",
            "us_per_token": round(us_tok, 2), "us_per_layer": round(us_tok / STACK_LAYERS, 2),
            "sustained_hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "outputs_finite": finite,
            "tokens_0_255_equal_layer_by_layer_calls": same}


# The K3 LatentMoE layer: hidden 7168, latent 3584, 896 experts top-16 of intermediate 3072
# (MXFP4, at the latent width), two bf16 shared experts (intermediate 6144 together), SiTU
# betas 4 and 25, the latent RMSNorm, routed_scale 1.
K3_E, K3_K, K3_I, K3_L, K3_SI = 896, 16, 3072, 3584, 6144
K3_KERNELS = ["k1_router_bset", "k1_zdown", "k2_gateup", "k3_down", "k4_up"]


def k3_kernel_bytes(U, T):
    """Algorithmic HBM bytes per launch of the latent decode kernels at one token (k4_up
    works out the latent norm itself there): k1 the router, zdown the down projection, k2
    the shared experts' and the unique experts' gate/up weights, k3 the unique experts'
    down weights, k4 the up projection and the shared experts' down weights; activations
    in and out included."""
    xb = T * H * 2
    ex = K3_I * K3_L // 2 + K3_I * K3_L // 32
    return dict(zip(K3_KERNELS, (
        K3_E * H * 4 + K3_E * 4 + xb,
        K3_L * H * 2 + xb,
        2 * K3_SI * H * 2 + U * 2 * ex + 2 * T * K3_E * 4,
        U * ex + T * K3_L * 4,
        H * K3_L * 2 + H * K3_SI * 2 + T * H * 4)))


def k3_leg(torch, k3x, steps, warmup, nrot=2):
    """Decode b=1 through the K3 LatentMoE layer shape (15.7 GB of experts per layer),
    rotating over `nrot` layers so every call reads its weights from HBM; bf16 tokens from
    a pool of 64.  Reports microseconds per token, the per-kernel HIP-event durations and
    the dominant kernel's fraction of the HBM peak."""
    cfg = k3x.make_cfg(H, K3_E, K3_K, K3_I, 2, 1, 1.0, latent=K3_L, latent_norm=1,
                       rms_eps=1e-5, situ_b1=4.0, situ_b2=25.0)
    layers = [k3x.MoELayer.synthetic(cfg, seed=40 + j) for j in range(nrot)]
    n_pool = 64
    xs = k3x.synth_normal_f32(n_pool * H, k3x.synth_key(40, 0, k3x.STREAM_X, 100))
    xpool = torch.from_numpy(xs.reshape(n_pool, H)).cuda().to(torch.bfloat16).contiguous()
    out = torch.empty((1, H), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream
    row = xpool.stride(0) * 2

    def step(i):
        layers[i % nrot].forward(out.data_ptr(), xpool.data_ptr() + (i % n_pool) * row, 1,
                                 k3x.K3X_BF16, stream=sh)

    with torch.cuda.stream(stream):
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            step(warmup + i)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    for l in layers:
        l.set_timing(True)
    per = {n: [] for n in K3_KERNELS}
    with torch.cuda.stream(stream):
        for i in range(steps):
            step(i)
            for n, v in zip(K3_KERNELS, layers[i % nrot].last_ms()):
                per[n].append(v)
    for l in layers:
        l.set_timing(False)
        l.check()
    avg = {n: float(np.mean(v)) for n, v in per.items()}
    kb = k3_kernel_bytes(U=K3_K, T=1)
    dom = max(avg, key=lambda n: avg[n])
    achieved = kb[dom] / (avg[dom] * 1e-3) / 1e9
    total = sum(kb.values())
    finite = bool(torch.isfinite(out).all().item())
    for l in layers:
        l.close()
    del xpool, out
    torch.cuda.empty_cache()
    return {"workload": "K3 LatentMoE decode b=1: hidden 7168, latent 3584, 896 experts "
                        "top-16, inter 3072 MXFP4, 2 bf16 shared experts, SiTU 4/25, "
                        f"latent RMSNorm; {nrot} layers rotated",
            "us_per_token": round(wall_ms * 1e3, 2),
            "layer_bytes": total,
            "layer_hbm_gbs": round(total / (wall_ms * 1e-3) / 1e9, 1),
            "kernel_avg_us": {n: round(v * 1e3, 2) for n, v in avg.items()},
            "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes_per_launch": kb[dom]},
            "outputs_finite": finite, "steps": steps}


def k3_prefill_leg(torch, k3x, reps=3):
    """Prefill of one 2048-token chunk of bf16 N(0,1) activations through the K3 LatentMoE
    shape with Zipf-skewed routing (alpha 1.0, s 1.1).  Algorithmic bytes: the weight bytes
    of the experts the chunk uses, the shared experts, the latent projections and the
    router, once, plus the activations in and out.  FLOPs: 2 per multiply-add of the
    routed experts, the shared experts, the two projections and the router."""
    T = PREFILL_T
    cfg = k3x.make_cfg(H, K3_E, K3_K, K3_I, 2, 1, 1.0, latent=K3_L, latent_norm=1,
                       rms_eps=1e-5, situ_b1=4.0, situ_b2=25.0)
    layer = k3x.MoELayer.synthetic(cfg, seed=43, zipf_alpha=1.0)
    xs = k3x.synth_normal_f32(T * H, k3x.synth_key(43, 0, k3x.STREAM_X, 5))
    x = torch.from_numpy(xs.reshape(T, H)).cuda().to(torch.bfloat16).contiguous()
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, K3_K), dtype=torch.int32, device="cuda")
    wt = torch.empty((T, K3_K), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream

    def run():
        layer.forward(out.data_ptr(), x.data_ptr(), T, k3x.K3X_BF16, 0, idx.data_ptr(),
                      wt.data_ptr(), stream=sh)

    with torch.cuda.stream(stream):
        run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    used = int(torch.unique(idx).numel())
    ex = 3 * (K3_I * K3_L // 2 + K3_I * K3_L // 32)
    layer_bytes = (used * ex + 3 * K3_SI * H * 2 + 2 * K3_L * H * 2 + K3_E * H * 4 +
                   T * H * 2 + T * H * 4)
    flops = 2.0 * T * (K3_K * 3 * K3_I * K3_L + 3 * K3_SI * H + 2 * K3_L * H + K3_E * H)
    finite = bool(torch.isfinite(out).all().item())
    layer.close()
    del x, out, idx, wt
    torch.cuda.empty_cache()
    return {"workload": f"K3 LatentMoE prefill {T} bf16 tokens, Zipf-skewed routing "
                        "(alpha 1.0, s 1.1)",
            "tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_chunk": round(ms, 3),
            "experts_used": used,
            "hbm_gbs": round(layer_bytes / (ms * 1e-3) / 1e9, 1),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "mfma_frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / 2500.0, 4),
            "outputs_finite": finite, "reps": reps}


def trunk_leg(torch, k3x, reps=48, nrot=4):
    """bf16 trunk matrices of 7168 x 7168 (103 MB each, the size class of the K3 trunk's
    projections; `nrot` of them used in turn so that no call finds its matrix in the
    256 MB last-level cache) applied to 1 bf16 row (the GEMV: HBM-bound, bytes = the
    matrix) and to 2048 rows (the GEMM: 2 * 2048 * 7168^2 FLOP; bf16 input is one B
    column per row)."""
    n = 7168
    trs = []
    for j in range(nrot):
        w = k3x.synth_normal_bf16(n * n, k3x.synth_key(77, j, k3x.STREAM_SH1, 0), 0.0, 0.02)
        trs.append(k3x.Trunk(w.reshape(n, n)))
    rec = {"workload": f"bf16 trunk product, 7168 x 7168 weights, {nrot} matrices in turn"}
    stream = torch.cuda.Stream()
    for T in (1, 2048):
        xs = k3x.synth_normal_f32(T * n, k3x.synth_key(77, 0, k3x.STREAM_X, T))
        x = torch.from_numpy(xs.reshape(T, n)).cuda().to(torch.bfloat16).contiguous()
        y = torch.empty((T, n), dtype=torch.float32, device="cuda")
        r = reps if T == 1 else 8
        with torch.cuda.stream(stream):
            for i in range(nrot):
                trs[i].apply(y.data_ptr(), n, x.data_ptr(), k3x.K3X_BF16, n, T, stream.cuda_stream)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(r):
                trs[i % nrot].apply(y.data_ptr(), n, x.data_ptr(), k3x.K3X_BF16, n, T,
                                    stream.cuda_stream)
            e1.record(stream)
            torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / r
        if T == 1:
            gbs = n * n * 2 / (us * 1e-6) / 1e9
            rec["gemv_t1_us"] = round(us, 2)
            rec["gemv_t1_gbs"] = round(gbs, 1)
            rec["gemv_t1_hbm_frac"] = round(gbs / HBM_PEAK_GBS, 4)
        else:
            tf = 2.0 * T * n * n / (us * 1e-6) / 1e12
            rec["gemm_t2048_us"] = round(us, 1)
            rec["gemm_t2048_tflops"] = round(tf, 1)
            rec["gemm_t2048_bf16_peak_frac"] = round(tf / 2500.0, 4)
        del x, y
    for tr in trs:
        tr.close()
    torch.cuda.empty_cache()
    return rec


def k3_multi_leg(torch, k3x, tokens=(2, 4, 8), steps=60, warmup=10, nrot=2):
    """Decode calls of several bf16 tokens through the K3 LatentMoE layer shape with
    Zipf-skewed routing (alpha 1.0, s 1.1), `nrot` layers in turn: microseconds per call
    for each token count."""
    cfg = k3x.make_cfg(H, K3_E, K3_K, K3_I, 2, 1, 1.0, latent=K3_L, latent_norm=1,
                       rms_eps=1e-5, situ_b1=4.0, situ_b2=25.0)
    layers = [k3x.MoELayer.synthetic(cfg, seed=60 + j, zipf_alpha=1.0) for j in range(nrot)]
    n_pool = 64
    rec = {"workload": "K3 LatentMoE decode, several bf16 tokens a call, Zipf-skewed routing "
                       f"(alpha 1.0, s 1.1), {nrot} layers in turn", "us_per_call": {}}
    stream = torch.cuda.Stream()
    for T in tokens:
        xs = k3x.synth_normal_f32(n_pool * T * H, k3x.synth_key(60, 0, k3x.STREAM_X, T))
        xpool = torch.from_numpy(xs.reshape(n_pool, T, H)).cuda().to(torch.bfloat16).contiguous()
        out = torch.empty((T, H), dtype=torch.float32, device="cuda")
        with torch.cuda.stream(stream):
            for i in range(warmup + steps):
                if i == warmup:
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                layers[i % nrot].forward(out.data_ptr(), xpool[i % n_pool].data_ptr(), T,
                                         k3x.K3X_BF16, stream=stream.cuda_stream)
            torch.cuda.synchronize()
        rec["us_per_call"][str(T)] = round((time.perf_counter() - t0) * 1e6 / steps, 1)
        # one call of T tokens against the same tokens one call each (the T = 1 path):
        # the same experts, outputs within 1e-5 relative L2 (only the accumulation order
        # of the two paths differs); the oracle's parity at this shape is a GPU test
        idx = torch.empty((T, K3_K), dtype=torch.int32, device="cuda")
        wt = torch.empty((T, K3_K), dtype=torch.float32, device="cuda")
        layers[0].forward(out.data_ptr(), xpool[0].data_ptr(), T, k3x.K3X_BF16, 0,
                          idx.data_ptr(), wt.data_ptr())
        one = torch.empty((1, H), dtype=torch.float32, device="cuda")
        i1 = torch.empty((1, K3_K), dtype=torch.int32, device="cuda")
        w1 = torch.empty((1, K3_K), dtype=torch.float32, device="cuda")
        err, same_idx = 0.0, True
        for t in range(T):
            layers[0].forward(one.data_ptr(), xpool[0][t:t + 1].data_ptr(), 1, k3x.K3X_BF16, 0,
                              i1.data_ptr(), w1.data_ptr())
            torch.cuda.synchronize()
            same_idx = same_idx and bool(torch.equal(i1[0], idx[t]))
            d = (one[0].double() - out[t].double()).norm() / out[t].double().norm()
            err = max(err, float(d))
        rec.setdefault("vs_single_token_calls", {})[str(T)] = {
            "same_experts": same_idx, "max_rel_l2": float(f"{err:.3e}"),
            "finite": bool(torch.isfinite(out).all().item())}
        del xpool, out
    for l in layers:
        l.check()
        l.close()
    torch.cuda.empty_cache()
    return rec


def verify_leg(torch, k3x, steps=100, warmup=10, nrot=4):
    """Speculative verification, T = 8 tokens per call, through the full-size K2-class
    layer with Zipf-skewed routing (alpha 1.0, s 1.1): microseconds per call and the HBM
    fraction of the call's algorithmic bytes (U unique experts x 23.4 MB + the shared
    expert and the router), `nrot` layers in turn."""
    T = 8
    cfg = k3x.make_cfg(H, E, K, I, 1, 1, 2.5)
    layers = [k3x.MoELayer.synthetic(cfg, seed=50 + j, zipf_alpha=1.0) for j in range(nrot)]
    n_pool = 64
    xs = k3x.synth_normal_f32(n_pool * T * H, k3x.synth_key(50, 0, k3x.STREAM_X, 8))
    xpool = torch.from_numpy(xs.reshape(n_pool, T, H)).cuda().to(torch.bfloat16).contiguous()
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((T, K), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    uniq = []

    def step(i, routing=False):
        layers[i % nrot].forward(out.data_ptr(), xpool[i % n_pool].data_ptr(), T, k3x.K3X_BF16,
                                 0, idx.data_ptr() if routing else 0,
                                 wt.data_ptr() if routing else 0, stream=stream.cuda_stream)

    with torch.cuda.stream(stream):
        for i in range(n_pool):                 # the pool's unique-expert counts
            step(i, routing=True)
            uniq.append(int(torch.unique(idx).numel()))
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            step(warmup + i)
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) * 1e6 / steps
    for l in layers:
        l.check()
        l.close()
    del xpool, out, idx, wt
    torch.cuda.empty_cache()
    u = float(np.mean([uniq[(warmup + i) % n_pool] for i in range(steps)]))
    nbytes = u * B_EXPERT + B_SHARED + B_ROUTER + T * H * 2 + T * H * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": "verify T=8 bf16 tokens per call, full-size K2-class layer, Zipf-skewed "
                        f"routing (alpha 1.0, s 1.1), {nrot} layers in turn",
            "us_per_call": round(us, 2), "unique_experts_mean": round(u, 2),
            "algorithmic_mb_per_call": round(nbytes / 1e6, 1),
            "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary (FETCH_SIZE and
    WRITE_SIZE runs scaled by a plain copy's readings), or None."""
    path = os.path.join(ROOT, "profiles", "decode_b1_hbm_traffic.md")
    try:
        for line in open(path):
            f = line.split()
            if len(f) == 3 and f[0] == "traffic_bytes_per_launch" and f[1] == kernel:
                return int(f[2])
    except OSError:
        pass
    return None


def _host():
    """The compiled reference for this host (its AVX-512 build where the host has
    x86-64-v4, what its -march=native build selects there, else the AVX2 build), or None
    (then the oracle port is timed), and the host facts every CPU baseline reports."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol
    import platform

    isa = "x86-64-v4" if ol.ref("x86-64-v4") is not None else "x86-64-v3"
    ref = ol.ref(isa)
    kind = "reference" if ref is not None else "port"
    cores = int(ol.oracle().ko_threads())
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    libc = platform.libc_ver()
    info = {"cores": cores, "kind": kind,
            "isa": isa if kind == "reference" else "x86-64-v3 (oracle port)",
            "build": "gcc -O3 -fopenmp -ffp-contract=off -march=" + isa
                     + " (oracle/Makefile, the reference's flags but -march)",
            "cpu_model": cpu_model, "glibc": f"{libc[0]} {libc[1]}"}
    return ref, info


def _bank(L, experts):
    """The experts' arrays of layer L in the reference's layout, as the harness's bank
    (the arrays are kept alive by the returned dict)."""
    import oracle_lib as ol
    bank = (ol.KoExpert * L.E)()
    keep = {}
    for e in experts:
        d = {k: v.copy() for k, v in L.expert(e).items()}
        keep[e] = d
        for k in ("p1", "s1", "p3", "s3", "p2", "s2"):
            setattr(bank[e], k, d[k].ctypes.data_as(ol.U8P))
    return bank, keep


def _route(L, x):
    """Every row's top-k experts by the oracle's router (to know which to generate)."""
    import oracle_lib as ol
    idx = np.empty((x.shape[0], L.K), np.int32)
    wt = np.empty((x.shape[0], L.K), np.float32)
    for t in range(x.shape[0]):
        xt = np.ascontiguousarray(x[t])
        ol.oracle().ko_router(ol.ptr(idx[t], ol.I32P), ol.ptr(wt[t], ol.F32P),
                              ol.ptr(xt, ol.F32P), ol.ptr(L.gate, ol.F32P),
                              ol.ptr(L.bias, ol.F32P), L.H, L.E, L.K, L.renorm,
                              L.routed_scale)
    return idx


def _k2_args(L, bank):
    import oracle_lib as ol
    return (L.H, L.E, L.K, L.I, L.I * L.n_shared, L.routed_scale, L.renorm,
            ol.ptr(L.gate, ol.F32P), ol.ptr(L.bias, ol.F32P), bank, ol.ptr(L.sh1, ol.U16P),
            ol.ptr(L.sh3, ol.U16P), ol.ptr(L.sh2, ol.U16P))


def cpu_baseline(n_tokens=24, min_seconds=10.0):
    """The decode layer on the host CPU over a bounded sample of tokens (same seeded
    layer): the reference's k3_moe work per token (refdrv_k2_tokens), median per token."""
    t_setup = time.perf_counter()
    ref, info = _host()               # puts the test infrastructure on the path
    import oracle_lib as ol
    import synth

    L = synth.full(seed=1)
    x = L.x(n_tokens, bf16=True, stream_sub=7)
    need = sorted(set(_route(L, x).ravel().tolist()))
    bank, keep = _bank(L, need)
    out = np.empty((1, H), np.float32)
    ii = np.empty((1, K), np.int32)
    ww = np.empty((1, K), np.float32)
    setup_s = time.perf_counter() - t_setup   # weights generated on the host, untimed
    times = []
    t_start = time.perf_counter()
    while True:
        for t in range(n_tokens):
            xt = np.ascontiguousarray(x[t:t + 1])
            t0 = time.perf_counter()
            if ref is not None:
                ref.refdrv_k2_tokens(ol.ptr(out, ol.F32P), ol.ptr(xt, ol.F32P), 1,
                                     *_k2_args(L, bank), ol.ptr(ii, ol.I32P),
                                     ol.ptr(ww, ol.F32P))
            else:
                L.oracle_moe(xt)
            times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= min_seconds:
            break
    us = float(np.median(times) * 1e6)
    rec = {"value": round(us, 1), "unit": "us/token"}
    rec.update(info)
    rec["setup_s"] = round(setup_s, 1)
    rec["sample"] = (f"{len(times)} layer calls over {n_tokens} distinct bf16 tokens of the "
                     f"same seeded layer ({len(need)} experts generated), median per token, "
                     f"OpenMP threads {info['cores']}")
    return rec


def cpu_baseline_prefill(min_seconds=10.0, n_tokens=64):
    """The prefill leg's layer and chunk on the host CPU over a bounded sample: the
    chunk's first n_tokens rows (64: one of the sub-chunks in which the reference's
    k3_moe_prefill routes, fetches each unique expert once and applies it to every token
    that chose it), as one prefill call of the reference's kernels (refdrv_k2_prefill,
    with the shared expert's batched products); median over calls, as tokens/s."""
    t_setup = time.perf_counter()
    ref, info = _host()               # puts the test infrastructure on the path
    import oracle_lib as ol
    import synth

    L = synth.full(seed=3, zipf_alpha=1.0)
    x = L.x(n_tokens, bf16=True, stream_sub=5)      # rows 0 .. n_tokens - 1 of the chunk
    need = sorted(set(_route(L, x).ravel().tolist()))
    bank, keep = _bank(L, need)
    out = np.empty((n_tokens, H), np.float32)
    ii = np.empty((n_tokens, K), np.int32)
    ww = np.empty((n_tokens, K), np.float32)
    setup_s = time.perf_counter() - t_setup   # weights generated on the host, untimed
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        if ref is not None:
            ref.refdrv_k2_prefill(ol.ptr(out, ol.F32P), ol.ptr(x, ol.F32P), n_tokens,
                                  *_k2_args(L, bank), ol.ptr(ii, ol.I32P), ol.ptr(ww, ol.F32P))
        else:
            L.oracle_moe(x, prefill=True)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= min_seconds and len(times) >= 3:
            break
    s = float(np.median(times))
    rec = {"value": round(n_tokens / s, 1), "unit": "tokens/s",
           "ms_per_sample": round(s * 1e3, 2)}
    rec.update(info)
    rec["setup_s"] = round(setup_s, 1)
    rec["sample"] = (f"rows 0-{n_tokens - 1} of the 2048-token chunk (one 64-position "
                     f"sub-chunk of the reference's prefill; {len(need)} unique experts, "
                     f"generated), {len(times)} calls, median, OpenMP threads {info['cores']}")
    return rec


def cpu_baseline_stack(min_seconds=10.0, n_tokens=2):
    """The stack leg's eight layers on the host CPU for the stack's first n_tokens
    tokens: per layer h = h + MoE(RMSNorm(h)) with the reference's k3_rmsnorm and k3_moe
    work (refdrv_k2_norm_layer); median time of a token through the eight layers."""
    t_setup = time.perf_counter()
    ref, info = _host()               # puts the test infrastructure on the path
    import oracle_lib as ol
    import synth

    Ls = [synth.full(seed=10 + l, layer=l) for l in range(STACK_LAYERS)]
    norms = [synth.normal_f32(H, synth.key(10 + l, l, synth.S_NORM), 1.0, 0.1)
             for l in range(STACK_LAYERS)]
    x = Ls[0].x(n_tokens, bf16=False, stream_sub=7)    # the stack leg's first tokens
    ii = np.empty((1, K), np.int32)
    ww = np.empty((1, K), np.float32)

    def layer_step(l, bank, h):
        if ref is not None:
            rc = ref.refdrv_k2_norm_layer(ol.ptr(h, ol.F32P), h.shape[0],
                                          ol.ptr(norms[l], ol.F32P), 1e-5,
                                          *_k2_args(Ls[l], bank), ol.ptr(ii, ol.I32P),
                                          ol.ptr(ww, ol.F32P))
            assert rc == 0
            return h
        hin = np.empty_like(h)
        for t in range(h.shape[0]):
            ol.oracle().ko_rmsnorm(ol.ptr(hin[t], ol.F32P),
                                   ol.ptr(np.ascontiguousarray(h[t]), ol.F32P),
                                   ol.ptr(norms[l], ol.F32P), H, 1e-5)
        return h + Ls[l].oracle_moe(hin)[0]

    # the experts each layer's routing needs, layer by layer (a layer's input is the
    # previous layer's output)
    banks, n_exp = [], 0
    h = x.copy()
    for l in range(STACK_LAYERS):
        hin = np.empty_like(h)
        for t in range(n_tokens):
            ol.oracle().ko_rmsnorm(ol.ptr(hin[t], ol.F32P),
                                   ol.ptr(np.ascontiguousarray(h[t]), ol.F32P),
                                   ol.ptr(norms[l], ol.F32P), H, 1e-5)
        need = sorted(set(_route(Ls[l], hin).ravel().tolist()))
        n_exp += len(need)
        banks.append(_bank(Ls[l], need))
        for t in range(n_tokens):
            h[t:t + 1] = layer_step(l, banks[l][0], np.ascontiguousarray(h[t:t + 1]))
    setup_s = time.perf_counter() - t_setup   # weights generated on the host, untimed
    times = []
    t_start = time.perf_counter()
    while True:
        for t in range(n_tokens):
            ht = x[t:t + 1].copy()            # the layers update their rows in place
            t0 = time.perf_counter()
            for l in range(STACK_LAYERS):
                ht = layer_step(l, banks[l][0], ht)
            times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= min_seconds:
            break
    us = float(np.median(times) * 1e6)
    rec = {"value": round(us, 1), "unit": "us/token", "us_per_layer": round(us / STACK_LAYERS, 1)}
    rec.update(info)
    rec["setup_s"] = round(setup_s, 1)
    rec["sample"] = (f"the stack's tokens 0-{n_tokens - 1} through its {STACK_LAYERS} layers "
                     f"({n_exp} experts generated), {len(times)} passes, median per token, "
                     f"OpenMP threads {info['cores']}")
    return rec


def copy_calibration(torch, mib, reps):
    """A plain device-to-device copy of a known size: FETCH_SIZE and WRITE_SIZE read
    for it give the factor between those counters and bytes moved."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / reps
    print(json.dumps({"copy_bytes": n, "reps": reps, "ms_per_copy": round(ms, 4),
                      "copy_gbs": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 2048-token prefill leg")
    ap.add_argument("--no-stack", action="store_true", help="skip the 8-layer stack leg")
    ap.add_argument("--no-k3", action="store_true", help="skip the K3 LatentMoE decode leg")
    ap.add_argument("--no-trunk", action="store_true", help="skip the trunk product leg")
    ap.add_argument("--no-verify", action="store_true", help="skip the T=8 verify leg")
    ap.add_argument("--trunk-only", action="store_true",
                    help="only run the trunk product leg and print its record")
    ap.add_argument("--k3-only", action="store_true",
                    help="only run the K3 LatentMoE decode leg and print its record")
    ap.add_argument("--stack-only", action="store_true",
                    help="only run the 8-layer stack leg and print its record")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only run the prefill leg and print its record")
    ap.add_argument("--k3-multi-only", action="store_true",
                    help="only run the K3 LatentMoE several-token decode leg")
    ap.add_argument("--verify-only", action="store_true",
                    help="only run the T=8 verify leg and print its record")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only time a plain device copy of MIB MiB (the reference kernel for "
                         "the HBM byte counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this library has no multi-GPU path "
              "(collectives and sharding are out of scope); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "no GPU visible"
    if args.calibrate_copy:
        copy_calibration(torch, args.calibrate_copy, max(args.steps, 1))
        return
    if args.prefill_only:
        print(json.dumps(prefill_leg(torch, load_k3x())), flush=True)
        return
    if args.stack_only:
        print(json.dumps(stack_leg(torch, load_k3x())), flush=True)
        return
    if args.trunk_only:
        print(json.dumps(trunk_leg(torch, load_k3x())), flush=True)
        return
    if args.k3_multi_only:
        print(json.dumps(k3_multi_leg(torch, load_k3x())), flush=True)
        return
    if args.verify_only:
        print(json.dumps(verify_leg(torch, load_k3x())), flush=True)
        return
    if args.k3_only:
        k = load_k3x()
        rec = k3_leg(torch, k, args.steps, args.warmup)
        if not args.no_prefill:
            rec["prefill"] = k3_prefill_leg(torch, k)
        print(json.dumps(rec), flush=True)
        return
    k3x = load_k3x()
    dev = torch.device("cuda:0")
    cfg = k3x.make_cfg(H, E, K, I, 1, 1, 2.5)
    t_build = time.perf_counter()
    # NROT layers of the same shape, used in turn: between two calls of one layer the
    # other layers stream about 860 MB, so no weight of the call is still in the 256 MB
    # last-level cache -- as in a model with many layers.
    layers = [k3x.MoELayer.synthetic(cfg, seed=1 + j, router_sigma=0.02, bias_sigma=0.1)
              for j in range(NROT)]
    build_s = (time.perf_counter() - t_build) / NROT
    n_pool = 64
    xs = k3x.synth_normal_f32(n_pool * H, k3x.synth_key(1, 0, k3x.STREAM_X, 100))
    xpool = torch.from_numpy(xs.reshape(n_pool, H)).to(dev).to(torch.bfloat16).contiguous()
    out = torch.empty((1, H), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    sh = stream.cuda_stream
    row = xpool.stride(0) * 2

    def step(i, rot=NROT):
        layers[i % rot].forward(out.data_ptr(), xpool.data_ptr() + (i % n_pool) * row, 1,
                                k3x.K3X_BF16, stream=sh)

    def timed(rot):
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                step(i, rot)
            torch.cuda.synchronize()
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            ev0.record(stream)
            for i in range(args.steps):
                step(args.warmup + i, rot)
            ev1.record(stream)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
        return (t1 - t0) * 1e3 / args.steps, ev0.elapsed_time(ev1) / args.steps

    wall_ms, gpu_ms = timed(NROT)
    warm_ms, _ = timed(1)

    # per-kernel durations: HIP events between the kernels, on the launch stream
    for l in layers:
        l.set_timing(True)
    names = KERNELS
    per = {n: [] for n in names}
    with torch.cuda.stream(stream):
        for i in range(args.steps):
            step(i)
            ms = layers[i % NROT].last_ms()
            for n, v in zip(names, ms):
                per[n].append(v)
    for l in layers:
        l.set_timing(False)
        l.check()               # no decode workgroup gave up waiting for the selection
    # how often the selection works a router logit out again as the reference's single
    # chain (a logit whose float the parallel sum does not prove and that could change the
    # selection or a selected weight): 512 further tokens, one synchronised call each,
    # outside the timed region
    n_ex = 512
    xe = k3x.synth_normal_f32(n_ex * H, k3x.synth_key(1, 0, k3x.STREAM_X, 101))
    xe = torch.from_numpy(xe.reshape(n_ex, H)).to(dev).to(torch.bfloat16).contiguous()
    tok_ex = logit_ex = 0
    with torch.cuda.stream(stream):
        for i in range(n_ex):
            layers[i % NROT].forward(out.data_ptr(), xe.data_ptr() + i * row, 1, k3x.K3X_BF16,
                                     stream=sh)
            c = layers[i % NROT].exact_count()
            tok_ex += int(c > 0)
            logit_ex += c
    del xe
    avg = {n: float(np.mean(v)) for n, v in per.items()}
    kb = kernel_bytes(U=K, T=1)
    dom = max(avg, key=lambda n: avg[n])
    achieved = kb[dom] / (avg[dom] * 1e-3) / 1e9
    layer_bytes = K * B_EXPERT + B_SHARED + B_ROUTER + H * 2 + H * 4
    rec = {
        "metric": "moe_layer_decode_b1_us_per_token",
        "value": round(wall_ms * 1e3, 2),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4-e2m1xe8m0 weights, bf16 mfma (hi+lo activations), fp32 accumulate",
        "data": "synthetic (seeded random weights and bf16 N(0,1) tokens)",
        "config": {"workload": "K2-class MoE layer decode b=1: hidden 7168, 384 experts top-8, "
                               "inter 2048 MXFP4, 1 bf16 shared expert",
                   "tokens_per_step": 1, "token_pool": n_pool, "layers_rotated": NROT,
                   "parallelism": "none (1 GPU)"},
        "layer_hbm_gbs": round(layer_bytes / (wall_ms * 1e-3) / 1e9, 1),
        "gpu_event_ms_per_step": round(gpu_ms, 5),
        "kernel_avg_us": {n: round(v * 1e3, 2) for n, v in avg.items()},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
                     "algorithmic_bytes_per_launch": kb[dom]},
        "layer_build_s": round(build_s, 2),
        "warm_one_layer_us_per_token": round(warm_ms * 1e3, 2),
        "router_exact_chain": {"tokens": n_ex, "tokens_with_a_chain": tok_ex,
                               "logits_worked_out": logit_ex},
    }
    for l in layers:
        l.close()
    del xpool, out
    torch.cuda.empty_cache()
    if not args.no_verify:
        rec["verify"] = verify_leg(torch, k3x)
    if not args.no_prefill:
        rec["prefill"] = prefill_leg(torch, k3x)
    if not args.no_stack:
        rec["stack"] = stack_leg(torch, k3x)
    if not args.no_k3:
        rec["k3_latent"] = k3_leg(torch, k3x, min(args.steps, 100), min(args.warmup, 10))
        if not args.no_prefill:
            rec["k3_latent"]["prefill"] = k3_prefill_leg(torch, k3x)
        rec["k3_latent"]["multi"] = k3_multi_leg(torch, k3x)
    if not args.no_trunk:
        rec["trunk"] = trunk_leg(torch, k3x)
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline(min_seconds=args.cpu_seconds)
        if "prefill" in rec:
            rec["prefill"]["cpu_baseline"] = cpu_baseline_prefill(min_seconds=args.cpu_seconds)
        if "stack" in rec:
            rec["stack"]["cpu_baseline"] = cpu_baseline_stack(min_seconds=args.cpu_seconds)
    else:
        rec["cpu_baseline"] = None
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
