"""CPU ORACLE for the motion encoder — test infrastructure only.

A restatement of talking-portrait.cpp's LIA motion encoder
(src/motion_enc.cpp:50-160 with the graph helpers of src/ops_common.h:12-42)
on the CPU: numpy for the orchestration, the fc chain and the blur, plain C
(oracle/mdec_ops.c: orc_conv2d_s) for the convolutions.  It is the checker of
the HIP encoder: only tests/ may import it; the shipped library never does.

The graph, as the reference builds it (weights already carry the load-time
folds of motion_ae_scale, src/motion_enc.cpp:14-45):

  x    = leaky(conv1x1(img, W_stem) + b_stem)                      conv0, 512^2
  for i = 1..7 (ResBlock, r -> r/2):
    x1 = leaky(conv3x3(x, W1, pad 1) + b1)
    x2 = leaky(conv3x3(blur(x1, k2, pad 2), W2, stride 2) + b2)
    sk = conv1x1(blur(x, ks, pad 1), Ws, stride 2)
    x  = x2 + sk                                                   conv_i
  appearance = conv4x4(x, W8)                                      conv8, 1x1
  lambda     = fc4(fc3(fc2(fc1(fc0(appearance)))))                 plain linears
  motion     = Q . lambda
  feats[j]   = conv_{6-j} pixel-major [r*r][C]

f16 mode (--ftype f16): a tensor kept f16 (file f16 and >= 4096 elements,
src/gguf_load.cpp:149-153) is a GEMM operand in f16, and the other operand is
rounded to f16 the way ggml's im2col / vec_dot convert it; blur kernels,
biases and the stem weight stay f32.  The bit-level rounding of ggml's
GEMM/direct-conv accumulation is parity unpinned (absent library); the
restatement is pinned to the upstream torch formulation in
tests/lia_torch.py (independent: no folds) and to closed forms.
"""
from __future__ import annotations

import math

import numpy as np

from . import mdec as M

# EncoderApp channels per ResBlock input / output (src/motion_enc.cpp:47-48)
ENC_IN = (32, 64, 128, 256, 512, 512, 512)
ENC_OUT = (64, 128, 256, 512, 512, 512, 512)
DIM = 512         # appearance / latent width
N_MOTION = 20     # motion coefficients (lambda)
RES = 512         # input image side


def weight_names(cin=ENC_IN, cout=ENC_OUT, dim=DIM, n_motion=N_MOTION):
    """(name, torch shape) of every encoder tensor (GGUF names)."""
    b0 = "enc.net_app.convs"
    v = [(f"{b0}.0.0.weight", (cin[0], 3, 1, 1)),
         (f"{b0}.0.1.bias", (cin[0],))]
    for i in range(1, len(cin) + 1):
        c, co = cin[i - 1], cout[i - 1]
        b = f"{b0}.{i}"
        v += [(f"{b}.conv1.0.weight", (c, c, 3, 3)),
              (f"{b}.conv1.1.bias", (c,)),
              (f"{b}.conv2.0.kernel", (4, 4)),
              (f"{b}.conv2.1.weight", (co, c, 3, 3)),
              (f"{b}.conv2.2.bias", (co,)),
              (f"{b}.skip.0.kernel", (4, 4)),
              (f"{b}.skip.1.weight", (co, c, 1, 1))]
    v.append((f"{b0}.{len(cin) + 1}.weight", (dim, cout[-1], 4, 4)))
    for i in range(5):
        o = n_motion if i == 4 else dim
        v += [(f"enc.fc.{i}.weight", (o, dim)), (f"enc.fc.{i}.bias", (o,))]
    v.append(("dec.direction.Q", (dim, n_motion)))
    return v


def motion_ae_scale(name, ne):
    """Load-time scale folding (src/motion_enc.cpp:14-45), encoder tensors
    and dec.direction.Q; ne is the ggml order (reversed torch shape)."""
    SQ2 = M.SQRT2
    if (name == "enc.net_app.convs.0.1.bias" or name.endswith(".conv1.1.bias")
            or name.endswith(".activate.bias")):
        return SQ2
    if not name.endswith(".weight"):
        return 1.0
    if name.startswith("dec.direction") or name.endswith("noise.weight"):
        return 1.0
    if name.endswith("modulation.weight"):
        return 1.0 / math.sqrt(float(ne[0]))
    if name.startswith("enc.fc."):
        return 1.0 / math.sqrt(float(ne[0]))
    conv = 1.0 / math.sqrt(float(ne[0] * ne[1] * ne[2]))
    if name == "enc.net_app.convs.0.0.weight" or name.endswith(".conv1.0.weight"):
        return conv * SQ2
    if name.endswith(".conv2.1.weight"):
        return conv
    if name.endswith(".skip.1.weight"):
        return conv / SQ2
    if name == "enc.net_app.convs.8.weight":
        return conv
    return 1.0


def load_weights(raw, keep_f16):
    """weights_t::load's numeric path for the encoder tensors (as
    mdec.load_weights): dev values, f16 flags."""
    dev, isf16 = {}, {}
    for name, (arr, f16_in_file) in raw.items():
        a = M._f32(arr)
        if f16_in_file:
            a = M.round_f16(a)
        s = motion_ae_scale(name, M.ggml_ne(a.shape))
        if s != 1.0:
            a = (a * np.float32(s)).astype(np.float32)
        big = keep_f16 and f16_in_file and a.size >= 4096
        isf16[name] = big
        dev[name] = M.round_f16(a) if big else a
    return dev, isf16


def blur(x, k, pad):
    """ggml_pad_ext + ggml_conv_2d_dw_direct with a 4x4 kernel
    (src/ops_common.h:36-42): x (C, H, W) -> (C, H + 2 pad - 3, W + 2 pad - 3),
    y = sum_{i,j} k[i, j] * xpad[:, oy + i, ox + j], f32 in (i, j) order."""
    x = M._f32(x)
    C, H, W = x.shape
    xp = np.zeros((C, H + 2 * pad, W + 2 * pad), np.float32)
    xp[:, pad:pad + H, pad:pad + W] = x
    OH, OW = H + 2 * pad - 3, W + 2 * pad - 3
    y = np.zeros((C, OH, OW), np.float32)
    for i in range(4):
        for j in range(4):
            y += np.float32(k[i, j]) * xp[:, i:i + OH, j:j + OW]
    return y


class Encoder:
    """Oracle motion encoder over a full set of raw encoder weights.

    cin/cout: ResBlock channel lists (the reference's ENC_IN/ENC_OUT;
    smaller lists give the same graph with fewer channels, for fast tests)."""

    def __init__(self, raw, ftype="f32", cin=ENC_IN, cout=ENC_OUT):
        assert ftype in ("f32", "f16")
        self.f16 = ftype == "f16"
        self.cin, self.cout = tuple(cin), tuple(cout)
        self.w, self.isf16 = load_weights(raw, self.f16)

    def _operand(self, x, wname):
        """the conv / GEMM operand as ggml builds it for weight `wname`"""
        return M.round_f16(x) if self.isf16[wname] else M._f32(x)

    def conv(self, x, wname, stride, pad):
        return M.conv2d_s(self._operand(x, wname), self.w[wname], stride, pad)

    def linear(self, x, wname, bname=None):
        """ggml_mul_mat(W, x) (+ b): f32 accumulation of f32 products"""
        xv = self._operand(x, wname).astype(np.float64)
        y = (self.w[wname].astype(np.float64) @ xv).astype(np.float32)
        if bname is not None:
            y = (y + self.w[bname]).astype(np.float32)
        return y

    @staticmethod
    def _act(y, b):
        return M.leaky((y + M._f32(b)[:, None, None]).astype(np.float32))

    def run(self, image):
        """image (3, 512, 512) f32 CHW in [-1, 1] -> dict with the taps
        menc.conv0..conv8, menc.fc0..fc4, appearance, lambda, motion and
        feats (list of (r*r, C) arrays, j = 0..6)."""
        b0 = "enc.net_app.convs"
        taps = {}
        x = self._act(self.conv(image, f"{b0}.0.0.weight", 1, 0), self.w[f"{b0}.0.1.bias"])
        taps["menc.conv0"] = x
        pyr = [x]
        for i in range(1, len(self.cin) + 1):
            b = f"{b0}.{i}"
            x1 = self._act(self.conv(x, f"{b}.conv1.0.weight", 1, 1), self.w[f"{b}.conv1.1.bias"])
            xb = blur(x1, self.w[f"{b}.conv2.0.kernel"], 2)
            x2 = self._act(self.conv(xb, f"{b}.conv2.1.weight", 2, 0), self.w[f"{b}.conv2.2.bias"])
            sb = blur(x, self.w[f"{b}.skip.0.kernel"], 1)
            sk = self.conv(sb, f"{b}.skip.1.weight", 2, 0)
            x = (x2 + sk).astype(np.float32)
            taps[f"menc.conv{i}"] = x
            pyr.append(x)
        wl = f"{b0}.{len(self.cin) + 1}.weight"
        app = self.conv(x, wl, 1, 0).reshape(-1)
        taps[f"menc.conv{len(self.cin) + 1}"] = app
        h = app
        for i in range(5):
            h = self.linear(h, f"enc.fc.{i}.weight", f"enc.fc.{i}.bias")
            taps[f"menc.fc{i}"] = h
        motion = self.linear(h, "dec.direction.Q")
        n = len(self.cin)
        feats = [np.ascontiguousarray(pyr[n - 1 - j].reshape(pyr[n - 1 - j].shape[0], -1).T)
                 for j in range(n)]
        return dict(taps=taps, appearance=app, **{"lambda": h}, motion=motion, feats=feats)
