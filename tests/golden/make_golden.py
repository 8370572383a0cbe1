"""Writes the small fixtures in this folder (run: python tests/golden/make_golden.py).

The expected outputs come from the reference's own ground-truth definitions,
evaluated here in float64 with torch's scaled_dot_product_attention:
  * causal FLARE, reference.py:37-43: for every t,
      z_t = SDPA(Q, K[:t+1], V[:t+1]);  y_t = SDPA(K_t, Q, z_t)
  * block-causal FLARE, semi_autoregressive/reference.py:575-596: per block g,
      z_g = SDPA(Q, K[:end_g], V[:end_g]);  y_block = SDPA(K_block, Q, z_g)
Inputs are seeded float32 values; the fixtures hold inputs, scale and outputs.
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def causal(q, k, v, scale):
    Q = q.double()[None].expand(k.shape[0], -1, -1, -1)
    K = k.double().permute(0, 2, 1, 3)
    V = v.double().permute(0, 2, 1, 3)
    Y = torch.empty(K.shape[0], K.shape[1], K.shape[2], V.shape[3], dtype=torch.float64)
    for t in range(K.shape[2]):
        z = F.scaled_dot_product_attention(Q, K[:, :, : t + 1], V[:, :, : t + 1], scale=scale)
        Y[:, :, t] = F.scaled_dot_product_attention(K[:, :, t : t + 1], Q, z, scale=scale)[:, :, 0]
    return Y.permute(0, 2, 1, 3)


def block_causal(q, k, v, block, scale):
    Q = q.double()[None].expand(k.shape[0], -1, -1, -1)
    K = k.double().permute(0, 2, 1, 3)
    V = v.double().permute(0, 2, 1, 3)
    Y = torch.empty(K.shape[0], K.shape[1], K.shape[2], V.shape[3], dtype=torch.float64)
    for g in range(K.shape[2] // block):
        s, e = g * block, (g + 1) * block
        z = F.scaled_dot_product_attention(Q, K[:, :, :e], V[:, :, :e], scale=scale)
        Y[:, :, s:e] = F.scaled_dot_product_attention(K[:, :, s:e], Q, z, scale=scale)
    return Y.permute(0, 2, 1, 3)


def main():
    cases = [
        ("ar_small", "ar", 0, (1, 24, 2, 16, 16, 16), {"chunk": 16}),
        ("ar_ragged", "ar", 1, (2, 45, 2, 32, 32, 16), {"chunk": 16}),
        ("prefill", "prefill", 2, (2, 19, 3, 16, 16, 32), {}),
        ("semi", "semi", 3, (1, 64, 2, 16, 16, 16), {"block": 16}),
    ]
    for name, kind, seed, (B, N, H, M, Dk, Dv), extra in cases:
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(H, M, Dk, generator=g)
        k = torch.randn(B, N, H, Dk, generator=g)
        v = torch.randn(B, N, H, Dv, generator=g)
        scale = 1.0 if kind == "prefill" else Dk ** -0.5
        if kind == "semi":
            y = block_causal(q, k, v, extra["block"], scale)
        else:
            y = causal(q, k, v, scale)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), kind=np.array(kind), q=q.numpy(), k=k.numpy(),
                            v=v.numpy(), y=y.numpy(), scale=np.array(scale),
                            **{kk: np.array(vv) for kk, vv in extra.items()})
        print("wrote", name, tuple(y.shape))


if __name__ == "__main__":
    main()
