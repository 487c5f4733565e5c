"""Independent torch-CPU formulation of FLOAT's flow-matching transformer
(DiT blocks with adaLN modulation, LayerNorm without affine, fused qkv
attention with a boolean band mask, tanh-GELU MLP, GLIDE timestep
embedding), written from the upstream module definitions in float64 with
torch's own primitives (F.layer_norm, F.scaled_dot_product_attention,
F.gelu(approximate="tanh")) and none of the reference's graph plumbing."""
import math

import torch
import torch.nn.functional as F


def modulate(x, shift, scale):
    return x * (1 + scale) + shift


def forward(raw, cfg, x60, cond, t):
    dt = torch.float64
    W = {k: torch.tensor(v[0], dtype=dt) for k, v in raw.items()}
    H, T, nh = cfg.dim_h, cfg.total, cfg.n_heads
    hd = H // nh

    def lin(x, name):
        return F.linear(x, W[name + ".weight"], W[name + ".bias"])

    half = cfg.t_freq_dim // 2
    freqs = torch.exp(-math.log(10000) * torch.arange(half, dtype=dt) / half)
    args = torch.tensor(t, dtype=dt) * freqs
    temb = torch.cat([torch.cos(args), torch.sin(args)])
    temb = lin(F.silu(lin(temb, "t_embedder.mlp.0")), "t_embedder.mlp.2")
    c = lin(torch.tensor(cond, dtype=dt), "c_embedder") + temb          # (3, T, H)
    x = lin(torch.tensor(x60, dtype=dt), "x_embedder.proj") + W["pos_embed"][0]
    x = x[None].repeat(3, 1, 1)
    idx = torch.arange(T)
    allowed = (idx[:, None] - idx[None, :]).abs() <= cfg.attn_window   # True = attend
    for i in range(cfg.depth):
        b = f"blocks.{i}"
        sh1, sc1, g1, sh2, sc2, g2 = lin(F.silu(c), f"{b}.adaLN_modulation.1").chunk(6, dim=-1)
        h = modulate(F.layer_norm(x, (H,), eps=cfg.ln_eps), sh1, sc1)
        qkv = lin(h, f"{b}.attn.qkv").reshape(3, T, 3, nh, hd).permute(2, 0, 3, 1, 4)
        o = F.scaled_dot_product_attention(qkv[0], qkv[1], qkv[2], attn_mask=allowed)
        x = x + g1 * lin(o.transpose(1, 2).reshape(3, T, H), f"{b}.attn.proj")
        h = modulate(F.layer_norm(x, (H,), eps=cfg.ln_eps), sh2, sc2)
        x = x + g2 * lin(F.gelu(lin(h, f"{b}.mlp.fc1"), approximate="tanh"), f"{b}.mlp.fc2")
    sh, sc = lin(F.silu(c), "decoder.adaLN_modulation.1").chunk(2, dim=-1)
    return lin(modulate(F.layer_norm(x, (H,), eps=cfg.ln_eps), sh, sc), "decoder.linear").numpy()
