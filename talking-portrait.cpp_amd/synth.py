"""Seeded synthetic decoder weights and inputs (no checkpoints are available).

Random-init weights of the LIA/StyleGAN decoder architecture, in the GGUF
tensor names and torch shapes the reference loads (src/motion_dec.cpp:17-29,
:659-1135), and the seeded inputs of the decoder workloads:

  weights  seed 1000: every .weight and dec.input.input ~ N(0,1) (raw, before
           the load-time Equal* scale folding); modulation.bias = 1.0
           (StyleGAN2 bias_init=1); other biases ~ N(0,1) * 0.1; blur and
           upsample kernels = [1,3,3,1] x [1,3,3,1] / 64 * 4.
  latents  seed 1001: w_t = s + Q alpha_t, s ~ N(0,1)^512, Q = QR-orthonormal
           512x20 from an N(0,1) matrix; alpha iid N(0,1) ("iid") or an AR(1)
           walk alpha_t = 0.95 alpha_{t-1} + 0.1 eps_t ("ar1"); "stress"
           scales alternate frames by 8 and 1/8.
  feats    seed 1002: feat_j ~ N(0,1), [r_j*r_j][OC_j] pixel-major.
Each tensor draws from its own PCG64 stream keyed by (seed, crc32(name)), so
values do not depend on generation order.

ftype "f16" emulates an f16 GGUF: tensors with >= 2 dims hold f16 values in
the file (rounded RNE here) and carry the F16_FILE flag.
"""
from __future__ import annotations

import zlib

import numpy as np

REF_IC = (512, 512, 512, 512, 256, 128, 64)
REF_OC = (512, 512, 512, 256, 128, 64, 32)
STYLE_DIM = 512


def _rng(seed, key):
    return np.random.Generator(np.random.PCG64([seed, zlib.crc32(key.encode())]))


def tensor_shapes(ic=REF_IC, oc=REF_OC):
    c0 = ic[0]
    v = [("dec.input.input", (1, c0, 4, 4)),
         ("dec.conv1.conv.weight", (1, c0, c0, 3, 3)),
         ("dec.conv1.conv.modulation.weight", (c0, STYLE_DIM)),
         ("dec.conv1.conv.modulation.bias", (c0,)),
         ("dec.conv1.activate.bias", (c0,))]
    for j in range(len(ic)):
        for i, cin in ((2 * j, ic[j]), (2 * j + 1, oc[j])):
            b = f"dec.convs.{i}"
            v += [(f"{b}.conv.weight", (1, oc[j], cin, 3, 3)),
                  (f"{b}.conv.modulation.weight", (cin, STYLE_DIM)),
                  (f"{b}.conv.modulation.bias", (cin,)),
                  (f"{b}.activate.bias", (oc[j],))]
            if i % 2 == 0:
                v.append((f"{b}.conv.blur.kernel", (4, 4)))
        f, r = f"dec.to_flows.{j}", f"dec.to_rgbs.{j}"
        v += [(f"{f}.conv.weight", (1, 3, oc[j], 1, 1)),
              (f"{f}.conv.modulation.weight", (oc[j], STYLE_DIM)),
              (f"{f}.conv.modulation.bias", (oc[j],)),
              (f"{f}.bias", (1, 3, 1, 1)),
              (f"{f}.upsample.kernel", (4, 4)),
              (f"{r}.conv.0.weight", (3, oc[j], 1, 1)),
              (f"{r}.conv.1.bias", (3,)),
              (f"{r}.bias", (1, 3, 1, 1)),
              (f"{r}.upsample.kernel", (4, 4))]
    return v


def blur_kernel():
    k1 = np.array([1, 3, 3, 1], np.float64)
    k = np.outer(k1, k1)
    return (k / k.sum() * 4.0).astype(np.float32)


def raw_weights(seed=1000, ftype="f32", ic=REF_IC, oc=REF_OC, flow_gain=1.0):
    """name -> (float32 array in torch shape, f16_in_file).  flow_gain scales
    the ToFlow conv weights (large displacements for the warp stress case)."""
    out = {}
    for name, shape in tensor_shapes(ic, oc):
        g = _rng(seed, name)
        if name.endswith(".kernel"):
            a = blur_kernel()
        elif name.endswith(".weight") or name == "dec.input.input":
            a = g.standard_normal(shape, dtype=np.float32)
            if name.startswith("dec.to_flows.") and name.endswith(".conv.weight"):
                a = (a * np.float32(flow_gain)).astype(np.float32)
        elif name.endswith(".modulation.bias"):
            a = np.ones(shape, np.float32)
        else:
            a = (g.standard_normal(shape, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
        f16 = ftype == "f16" and len(shape) >= 2
        if f16:
            a = a.astype(np.float16).astype(np.float32)
        out[name] = (np.ascontiguousarray(a), f16)
    return out


def latents(n, seed=1001, mode="iid"):
    """(n, 512) float32 decoder latents w = s + Q alpha."""
    g = _rng(seed, "latent")
    s = g.standard_normal(STYLE_DIM)
    q, _ = np.linalg.qr(g.standard_normal((STYLE_DIM, 20)))
    if mode == "iid":
        alpha = g.standard_normal((n, 20))
    else:
        alpha = np.empty((n, 20))
        alpha[0] = g.standard_normal(20)
        for t in range(1, n):
            alpha[t] = 0.95 * alpha[t - 1] + 0.1 * g.standard_normal(20)
    w = s[None, :] + alpha @ q.T
    if mode == "stress":
        scale = np.where(np.arange(n) % 2 == 0, 8.0, 1.0 / 8.0)
        w = w * scale[:, None]
    return np.ascontiguousarray(w.astype(np.float32))


def _blur_wrap(x, sigma):
    """separable gaussian blur (periodic) over the first two axes of x (r, r, C)"""
    rad = int(np.ceil(3 * sigma))
    k = np.exp(-0.5 * (np.arange(-rad, rad + 1) / sigma) ** 2)
    k /= k.sum()
    for ax in (0, 1):
        acc = np.zeros_like(x)
        for i, w in enumerate(k):
            acc += w * np.roll(x, i - rad, axis=ax)
        x = acc
    return x


def feats(seed=1002, oc=REF_OC, sigma=0.0):
    """per-stage warp features, feat_j (r_j*r_j, OC_j) float32, N(0,1).
    sigma > 0: spatially correlated like an encoder's conv features — i.i.d.
    N(0,1) blurred by a periodic gaussian of `sigma` pixels, then
    renormalised to zero mean and unit variance per channel."""
    out = []
    for j, c in enumerate(oc):
        r = 8 << j
        f = _rng(seed, f"feat{j}").standard_normal((r * r, c), dtype=np.float32)
        if sigma > 0:
            g = _blur_wrap(f.reshape(r, r, c).astype(np.float64), sigma)
            g = (g - g.mean(axis=(0, 1))) / g.std(axis=(0, 1))
            f = g.reshape(r * r, c).astype(np.float32)
        out.append(np.ascontiguousarray(f))
    return out


# decoder workloads:
#   iid    : the literal seeded configs — i.i.d. N(0,1) features, N(0,1)
#            ToFlow weights (flows saturate tanh: displacements up to the
#            whole map).  Chaotic: the gather amplifies any flow perturbation
#            by ~r/2 per stage, so only per-stage comparisons are meaningful.
#   smooth : encoder-like features (sigma = 2 px) and ToFlow weights x0.1 —
#            well-conditioned, used for end-to-end frame parity.
#   stress : i.i.d. features, ToFlow weights x8 (heavy zero padding), latents
#            scaled x8 / x1/8 on alternate frames (demodulation range).
WORKLOADS = {
    "iid": dict(flow_gain=1.0, sigma=0.0, latent_mode="ar1"),
    "smooth": dict(flow_gain=0.1, sigma=2.0, latent_mode="ar1"),
    "stress": dict(flow_gain=8.0, sigma=0.0, latent_mode="stress"),
}


def workload(name, n_frames, ftype="f32", ic=REF_IC, oc=REF_OC):
    """(raw weights, latents (n, 512), feats) of a named workload"""
    w = WORKLOADS[name]
    return (raw_weights(1000, ftype, ic, oc, flow_gain=w["flow_gain"]),
            latents(n_frames, 1001, w["latent_mode"]),
            feats(1002, oc, w["sigma"]))


# ---- motion encoder (src/motion_enc.cpp:47-160)
ENC_IN = (32, 64, 128, 256, 512, 512, 512)
ENC_OUT = (64, 128, 256, 512, 512, 512, 512)


def enc_tensor_shapes(cin=ENC_IN, cout=ENC_OUT, dim=STYLE_DIM, n_motion=20):
    """(name, torch shape) of every encoder tensor (GGUF names), with the
    decoder's dec.direction.Q the encoder also reads"""
    b0 = "enc.net_app.convs"
    v = [(f"{b0}.0.0.weight", (cin[0], 3, 1, 1)), (f"{b0}.0.1.bias", (cin[0],))]
    for i in range(1, len(cin) + 1):
        c, co, b = cin[i - 1], cout[i - 1], f"{b0}.{i}"
        v += [(f"{b}.conv1.0.weight", (c, c, 3, 3)), (f"{b}.conv1.1.bias", (c,)),
              (f"{b}.conv2.0.kernel", (4, 4)), (f"{b}.conv2.1.weight", (co, c, 3, 3)),
              (f"{b}.conv2.2.bias", (co,)), (f"{b}.skip.0.kernel", (4, 4)),
              (f"{b}.skip.1.weight", (co, c, 1, 1))]
    v.append((f"{b0}.{len(cin) + 1}.weight", (dim, cout[-1], 4, 4)))
    for i in range(5):
        v += [(f"enc.fc.{i}.weight", (n_motion if i == 4 else dim, dim)),
              (f"enc.fc.{i}.bias", (n_motion if i == 4 else dim,))]
    v.append(("dec.direction.Q", (dim, n_motion)))
    return v


def enc_raw_weights(seed=1004, ftype="f32", cin=ENC_IN, cout=ENC_OUT):
    """name -> (float32 array in torch shape, f16_in_file), seed 1004: every
    .weight ~ N(0,1) (raw, before the Equal* folds), biases ~ N(0,1) * 0.1,
    blur kernels [1,3,3,1] x [1,3,3,1] / 64 (downsampling Blur: no gain),
    dec.direction.Q QR-orthonormal (512 x 20)."""
    out = {}
    for name, shape in enc_tensor_shapes(cin, cout):
        g = _rng(seed, name)
        if name.endswith(".kernel"):
            a = (blur_kernel() / np.float32(4.0)).astype(np.float32)
        elif name == "dec.direction.Q":
            a = np.linalg.qr(g.standard_normal(shape))[0].astype(np.float32)
        elif name.endswith(".weight"):
            a = g.standard_normal(shape, dtype=np.float32)
        else:
            a = (g.standard_normal(shape, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
        f16 = ftype == "f16" and len(shape) >= 2 and not name.endswith(".kernel")
        if f16:
            a = a.astype(np.float16).astype(np.float32)
        out[name] = (np.ascontiguousarray(a), f16)
    return out


def image(seed=1005, res=512):
    """(3, res, res) float32 CHW in [-1, 1]: a smooth random field (a
    periodic gaussian blur of N(0,1), sigma 4 px) scaled and clipped like a
    normalised photograph"""
    f = _rng(seed, "image").standard_normal((res, res, 3))
    f = _blur_wrap(f, 4.0)
    f = f / f.std() * 0.5
    return np.ascontiguousarray(np.clip(f, -1.0, 1.0).transpose(2, 0, 1).astype(np.float32))


# ---- flow-matching transformer (src/fmt.cpp, src/pipeline.cpp:12-91)

class FmtConfig:
    """fmt_model's hyper-parameters at their defaults (src/fmt.h:9-17), as
    tpfm_default_config fills them; keyword arguments override"""

    def __init__(self, **kw):
        self.dim_h, self.depth, self.n_heads = 1024, 8, 8
        self.dim_w, self.dim_a, self.dim_e = 512, 512, 7
        self.chunk_frames, self.prev_frames = 50, 10
        self.attn_window, self.t_freq_dim, self.nfe = 2, 256, 10
        self.mlp_ratio, self.ln_eps = 4.0, 1e-6
        self.a_cfg, self.e_cfg, self.r_cfg = 2.0, 1.0, 1.0
        for k, v in kw.items():
            if not hasattr(self, k):
                raise AttributeError(k)
            setattr(self, k, v)
        self.total = self.chunk_frames + self.prev_frames

    @property
    def dim_c(self):
        return self.dim_w + self.dim_a + self.dim_e

    @property
    def dim_mlp(self):
        return int(self.dim_h * self.mlp_ratio)


def fmt_tensor_shapes(cfg):
    """(name, torch shape) of every FMT tensor in GGUF names
    (src/fmt.cpp:61-150); cfg: any object with FmtConfig's attributes"""
    H = cfg.dim_h
    v = [("t_embedder.mlp.0.weight", (H, cfg.t_freq_dim)), ("t_embedder.mlp.0.bias", (H,)),
         ("t_embedder.mlp.2.weight", (H, H)), ("t_embedder.mlp.2.bias", (H,)),
         ("c_embedder.weight", (H, cfg.dim_c)), ("c_embedder.bias", (H,)),
         ("x_embedder.proj.weight", (H, cfg.dim_w)), ("x_embedder.proj.bias", (H,)),
         ("pos_embed", (1, cfg.total, H))]
    for i in range(cfg.depth):
        b = f"blocks.{i}"
        for part, rows, cols in (("adaLN_modulation.1", 6 * H, H), ("attn.qkv", 3 * H, H), ("attn.proj", H, H),
                                 ("mlp.fc1", cfg.dim_mlp, H), ("mlp.fc2", H, cfg.dim_mlp)):
            v += [(f"{b}.{part}.weight", (rows, cols)), (f"{b}.{part}.bias", (rows,))]
    v += [("decoder.adaLN_modulation.1.weight", (2 * H, H)), ("decoder.adaLN_modulation.1.bias", (2 * H,)),
          ("decoder.linear.weight", (cfg.dim_w, H)), ("decoder.linear.bias", (cfg.dim_w,))]
    return v


def fmt_raw_weights(cfg, seed=1006, ftype="f32"):
    """name -> (float32 array in torch shape, f16_in_file) for an FMT of
    config `cfg` (FmtConfig or any object with its attributes), seed 1006:
    Linear weights ~ N(0,1)/sqrt(fan_in) (adaLN weights x0.5, so the gates
    and shifts are O(0.1-1) instead of the adaLN-Zero start), biases
    ~ N(0,1) * 0.02, pos_embed ~ N(0,1) * 0.1."""
    out = {}
    for name, shape in fmt_tensor_shapes(cfg):
        g = _rng(seed, name)
        a = g.standard_normal(shape, dtype=np.float32)
        if name.endswith(".weight"):
            a = a / np.float32(np.sqrt(shape[1]))
            if "adaLN" in name:
                a = a * np.float32(0.5)
        elif name == "pos_embed":
            a = a * np.float32(0.1)
        else:
            a = a * np.float32(0.02)
        a = a.astype(np.float32)
        f16 = ftype == "f16" and len(shape) >= 2 and name != "pos_embed"
        if f16:
            a = a.astype(np.float16).astype(np.float32)
        out[name] = (np.ascontiguousarray(a), f16)
    return out


def fmt_chunk_inputs(cfg, seed=1007):
    """one chunk's sampler inputs (src/pipeline.cpp:15-20): wr (dim_w,),
    prev_x (prev, dim_w), prev_wa (prev, dim_a), cond_audio (chunk, dim_a),
    x0 (chunk, dim_w) noise"""
    g = _rng(seed, "fmt_chunk")
    f = lambda *sh: np.ascontiguousarray(g.standard_normal(sh).astype(np.float32))
    P, CF = cfg.prev_frames, cfg.chunk_frames
    return dict(wr=f(cfg.dim_w), prev_x=f(P, cfg.dim_w), prev_wa=f(P, cfg.dim_a),
                cond_audio=f(CF, cfg.dim_a), x0=f(CF, cfg.dim_w))


def grid(n, lo, hi, seed=1003, jitter=0.0, res=None):
    """(n, 2) interleaved grid-sample coordinates ~ U(lo, hi) [+ U(-.5,.5)*jitter/res]."""
    g = _rng(seed, "grid")
    v = g.uniform(lo, hi, size=(n, 2))
    if jitter and res:
        v = v + g.uniform(-0.5, 0.5, size=(n, 2)) * jitter / res
    return np.ascontiguousarray(v.astype(np.float32))
