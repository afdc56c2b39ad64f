"""Helpers shared by the GPU tests: device forward through the C ABI, layer builders."""
import sys

import numpy as np


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev_forward(torch, k3x, layer, x, bf16=False, resid=None):
    """Run k3x_moe_forward on device copies; returns (out, idx, wt) on the host."""
    T, H = x.shape
    K = layer.cfg.topk
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    if bf16:
        xt = xt.to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    idx = torch.full((T, K), -7, dtype=torch.int32, device="cuda")
    wt = torch.empty((T, K), dtype=torch.float32, device="cuda")
    rp = 0
    if resid is not None:
        rt = torch.from_numpy(np.ascontiguousarray(resid)).cuda()
        rp = rt.data_ptr()
    s = torch.cuda.current_stream()
    layer.forward(out.data_ptr(), xt.data_ptr(), T, k3x.K3X_BF16 if bf16 else k3x.K3X_F32,
                  rp, idx.data_ptr(), wt.data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    layer.check()
    return out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()


def layer_cfg(k3x, L):
    """k3x_cfg of a synth.Layer (betas of 2^64 are passed as they are: SwiGLU)."""
    return k3x.make_cfg(L.H, L.E, L.K, L.I, L.n_shared, L.renorm, L.routed_scale,
                        latent=L.latent, latent_norm=L.latent_norm, rms_eps=L.rms_eps,
                        situ_b1=L.situ_b1, situ_b2=L.situ_b2)


def bank_layer(k3x, L):
    return k3x.MoELayer.from_bank(layer_cfg(k3x, L), L.gate, L.bias, L.all_experts(), L.sh1,
                                  L.sh3, L.sh2, down=L.down, up=L.up, latent_norm=L.lnorm)


def synth_layer(k3x, L):
    return k3x.MoELayer.synthetic(layer_cfg(k3x, L), seed=L.seed, layer=L.layer,
                                  router_sigma=L.router_sigma, bias_sigma=L.bias_sigma,
                                  zipf_alpha=L.zipf_alpha, zipf_s=L.zipf_s,
                                  scale_lo=L.scale_lo, scale_hi=L.scale_hi,
                                  shared_sigma=L.shared_sigma, trunk_sigma=L.trunk_sigma)
