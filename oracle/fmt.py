"""CPU ORACLE for the flow-matching transformer (FMT) — test infrastructure only.

A restatement of talking-portrait.cpp's FMT forward (src/fmt.cpp:44-205) and
its ODE chunk sampler (src/pipeline.cpp:12-91) in numpy (f32 storage, f64
GEMM accumulation).  It is the checker of the HIP FMT: only tests/ may import
it; the shipped library never does.

Forward, CFG-batched over B = 3 condition branches, T = prev + chunk tokens:
  t_emb  = W2 silu(W0 tfreq(t) + b0) + b2            tfreq = [cos(t f_k), sin(t f_k)]
  c      = Wc cond + bc + t_emb ;  sc = silu(c)      cond [B][T][dim_w+dim_a+dim_e]
  x      = Wx x60 + bx + pos                          (shared by the branches)
  block i (adaLN): (sh1, sc1, g1, sh2, sc2, g2) = Wm sc + bm
    h = norm(x) * sc1 + norm(x) + sh1 ; x += g1 * proj(attention(qkv(h)))
    h = norm(x) * sc2 + norm(x) + sh2 ; x += g2 * fc2(gelu_tanh(fc1(h)))
  final: (sh, scl) = Wf sc + bf ; v = Wl (norm(x) * scl + norm(x) + sh) + bl
attention: 8 heads, softmax(q k^T / sqrt(hd) + band mask), |i - j| <= window.

f16 checkpoints: tensors kept f16 (>= 4096 elements) are GEMM operands in
f16 with the activation rounded to f16 (ggml's mul_mat conversion); the
accumulation order of ggml's GEMMs is parity unpinned (absent library).
"""
from __future__ import annotations

import math

import numpy as np

from . import mdec as M


class Config:
    """fmt_model's hyper-parameters and their GGUF defaults (src/fmt.h:9-17)"""

    def __init__(self, **kw):
        self.dim_h, self.depth, self.n_heads = 1024, 8, 8
        self.dim_w, self.dim_a, self.dim_e = 512, 512, 7
        self.chunk_frames, self.prev_frames = 50, 10
        self.attn_window, self.t_freq_dim, self.nfe = 2, 256, 10
        self.mlp_ratio, self.ln_eps = 4.0, 1e-6
        self.a_cfg, self.e_cfg, self.r_cfg = 2.0, 1.0, 1.0
        for k, v in kw.items():
            assert hasattr(self, k), k
            setattr(self, k, v)
        self.total = self.chunk_frames + self.prev_frames

    @property
    def dim_c(self):
        return self.dim_w + self.dim_a + self.dim_e

    @property
    def dim_mlp(self):
        return int(self.dim_h * self.mlp_ratio)


def weight_names(cfg):
    """(name, torch shape) of every FMT tensor (GGUF names, src/fmt.cpp:61-150)"""
    H, T = cfg.dim_h, cfg.total
    v = [("t_embedder.mlp.0.weight", (H, cfg.t_freq_dim)), ("t_embedder.mlp.0.bias", (H,)),
         ("t_embedder.mlp.2.weight", (H, H)), ("t_embedder.mlp.2.bias", (H,)),
         ("c_embedder.weight", (H, cfg.dim_c)), ("c_embedder.bias", (H,)),
         ("x_embedder.proj.weight", (H, cfg.dim_w)), ("x_embedder.proj.bias", (H,)),
         ("pos_embed", (1, T, H))]
    for i in range(cfg.depth):
        b = f"blocks.{i}"
        v += [(f"{b}.adaLN_modulation.1.weight", (6 * H, H)), (f"{b}.adaLN_modulation.1.bias", (6 * H,)),
              (f"{b}.attn.qkv.weight", (3 * H, H)), (f"{b}.attn.qkv.bias", (3 * H,)),
              (f"{b}.attn.proj.weight", (H, H)), (f"{b}.attn.proj.bias", (H,)),
              (f"{b}.mlp.fc1.weight", (cfg.dim_mlp, H)), (f"{b}.mlp.fc1.bias", (cfg.dim_mlp,)),
              (f"{b}.mlp.fc2.weight", (H, cfg.dim_mlp)), (f"{b}.mlp.fc2.bias", (H,))]
    v += [("decoder.adaLN_modulation.1.weight", (2 * H, H)), ("decoder.adaLN_modulation.1.bias", (2 * H,)),
          ("decoder.linear.weight", (cfg.dim_w, H)), ("decoder.linear.bias", (cfg.dim_w,))]
    return v


def band_mask(T, w):
    """additive mask: 0 where row i attends col j (|i - j| <= w), -inf else
    (src/fmt.cpp:28-33, :152-156)"""
    i = np.arange(T)
    return np.where(np.abs(i[:, None] - i[None, :]) <= w, 0.0, -np.inf).astype(np.float32)


def t_freq(t, dim):
    """GLIDE sinusoidal timestep features (src/fmt.cpp:35-40, :168-174)"""
    half = dim // 2
    f = np.exp(-math.log(10000.0) * np.arange(half, dtype=np.float64) / half).astype(np.float32)
    a = (np.float32(t) * f).astype(np.float32)
    return np.concatenate([np.cos(a), np.sin(a)]).astype(np.float32)


def silu(x):
    x = M._f32(x)
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def gelu_tanh(x):
    x = M._f32(x).astype(np.float64)
    return (0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))).astype(np.float32)


def norm(x, eps):
    """ggml_norm over the last axis: (x - mean) / sqrt(var + eps)"""
    x = M._f32(x).astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    d = x - mu
    var = (d * d).mean(-1, keepdims=True)
    return (d / np.sqrt(var + eps)).astype(np.float32)


class FMT:
    def __init__(self, raw, cfg, ftype="f32"):
        self.cfg = cfg
        self.f16 = ftype == "f16"
        self.w, self.isf16 = {}, {}
        for name, (arr, f16_in_file) in raw.items():
            a = M._f32(arr)
            if f16_in_file:
                a = M.round_f16(a)
            big = self.f16 and f16_in_file and a.size >= 4096
            self.isf16[name] = big
            self.w[name] = M.round_f16(a) if big else a

    def linear(self, x, name):
        """y = x W^T + b over the last axis of x (ggml_mul_mat + add)"""
        W = self.w[name + ".weight"]
        xv = M.round_f16(x) if self.isf16[name + ".weight"] else M._f32(x)
        y = (xv.astype(np.float64) @ W.astype(np.float64).T).astype(np.float32)
        return (y + self.w[name + ".bias"]).astype(np.float32)

    def forward(self, x60, cond, t):
        """x60 (T, dim_w), cond (3, T, dim_c), t flow time -> v (3, T, dim_w)"""
        c, H = self.cfg, self.cfg.dim_h
        T, hd = c.total, H // c.n_heads
        te = self.linear(t_freq(t, c.t_freq_dim), "t_embedder.mlp.0")
        te = self.linear(silu(te), "t_embedder.mlp.2")
        cc = (self.linear(cond, "c_embedder") + te).astype(np.float32)
        sc = silu(cc)                                                   # (3, T, H)
        x = (self.linear(x60, "x_embedder.proj") + self.w["pos_embed"].reshape(T, H)).astype(np.float32)
        x = np.repeat(x[None], 3, axis=0)
        mask = band_mask(T, c.attn_window).astype(np.float64)
        scale = 1.0 / math.sqrt(hd)
        for i in range(c.depth):
            b = f"blocks.{i}"
            mod = self.linear(sc, f"{b}.adaLN_modulation.1")
            sh1, sc1, g1, sh2, sc2, g2 = (mod[..., k * H:(k + 1) * H] for k in range(6))
            h = norm(x, c.ln_eps)
            h = ((h * sc1 + h) + sh1).astype(np.float32)
            qkv = self.linear(h, f"{b}.attn.qkv")
            q, k, v = (qkv[..., j * H:(j + 1) * H].reshape(3, T, c.n_heads, hd).transpose(0, 2, 1, 3)
                       .astype(np.float64) for j in range(3))
            s = (q @ k.transpose(0, 1, 3, 2)) * np.float32(scale) + mask
            s = s - s.max(-1, keepdims=True)
            p = np.exp(s)
            p = p / p.sum(-1, keepdims=True)
            o = (p @ v).transpose(0, 2, 1, 3).reshape(3, T, H).astype(np.float32)
            x = (x + g1 * self.linear(o, f"{b}.attn.proj")).astype(np.float32)
            h = norm(x, c.ln_eps)
            h = ((h * sc2 + h) + sh2).astype(np.float32)
            m = self.linear(gelu_tanh(self.linear(h, f"{b}.mlp.fc1")), f"{b}.mlp.fc2")
            x = (x + g2 * m).astype(np.float32)
        fm = self.linear(sc, "decoder.adaLN_modulation.1")
        sh, scl = fm[..., :H], fm[..., H:]
        h = norm(x, c.ln_eps)
        h = ((h * scl + h) + sh).astype(np.float32)
        return self.linear(h, "decoder.linear")

    def cond_rows(self, wr, prev_wa, cond_audio, emotion):
        """the three CFG branches' condition rows (src/pipeline.cpp:22-36):
        [wr | wa | one-hot emotion]; branch 0 nulls the chunk's audio and the
        emotion, branch 2 (audio only) nulls the emotion"""
        c = self.cfg
        D, P, T = c.dim_w, c.prev_frames, c.total
        cond = np.zeros((3, T, c.dim_c), np.float32)
        cond[:, :, :D] = wr
        wa = np.concatenate([prev_wa, cond_audio], 0)
        for b in range(3):
            cond[b, :, D:D + c.dim_a] = wa
            if b == 0:
                cond[b, P:, D:D + c.dim_a] = 0.0
            if b == 1 and 0 <= emotion < c.dim_e:
                cond[b, :, D + c.dim_a + emotion] = 1.0
        return cond

    def sample_chunk(self, wr, prev_x, prev_wa, cond_audio, emotion, x0):
        """Euler ODE over nfe - 1 steps with the CFG combination
        (src/pipeline.cpp:38-91): returns the chunk's motion (chunk, dim_w)"""
        c = self.cfg
        P = c.prev_frames
        cond = self.cond_rows(wr, prev_wa, cond_audio, emotion)
        x = M._f32(x0).copy()
        ts = [np.float32(i / (c.nfe - 1)) for i in range(c.nfe)]
        for s in range(c.nfe - 1):
            x60 = np.concatenate([prev_x, x], 0).astype(np.float32)
            v = self.forward(x60, cond, float(ts[s]))
            u, fu, a = v[0], v[1], v[2]
            vc = ((u + np.float32(c.a_cfg) * (a - u)) + np.float32(c.e_cfg) * (fu - a)).astype(np.float32)
            dt = np.float32(ts[s + 1] - ts[s])
            x = (x + dt * vc[P:]).astype(np.float32)
        return x
