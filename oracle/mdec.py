"""CPU ORACLE for the motion decoder — test infrastructure only.

A restatement of talking-portrait.cpp's LIA/StyleGAN motion decoder
(src/motion_dec.cpp) on the CPU: numpy for the orchestration and the GEMMs,
plain C (oracle/mdec_ops.c, liboracle.so) for the patch's custom ops, the
prepare()-time derived tensors and the direct convolutions.  It is the
checker of the HIP implementation: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it; the shipped library never does.

Two graphs are restated, as the reference builds them:
  * decode_exact : the numerically conservative parity graph
                   (src/motion_dec.cpp:794-888): SP layout, direct convs,
                   map-side modulation, zero-stuff + flipped-W up-convs + blur.
  * decode_fast  : the batched channel-last generation graph
                   (src/motion_dec.cpp:889-1123): composed sub-pixel up-convs,
                   cf-im2col GEMMs, fold_into_weights decisions, SP direct-conv
                   stages from j = 5, and the f16 rounding points of --ftype f16.

numpy layout convention: a ggml tensor with ne = [n0, n1, n2, n3] is a
C-contiguous numpy array of shape (n3, n2, n1, n0).  So CL [C, N, B] is
(B, N, C) and SP [W, H, C, B] is (B, C, H, W).

Parity status: see the test files; functions whose rounding only the absent
ggml library could fix (GEMM accumulation order, conv_2d_direct internals)
are pinned to tolerance, not to bits.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

# stage channels (src/motion_dec.cpp:12-13)
REF_IC = (512, 512, 512, 512, 256, 128, 64)
REF_OC = (512, 512, 512, 256, 128, 64, 32)
STYLE_DIM = 512
SLOPE = 0.2
SQRT2 = 1.4142135623730951


# --------------------------------------------------------------------------
# native ops

def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/liboracle.so is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        sig = {
            "orc_round_f16": (None, [P, I64]),
            "orc_to_f16_bits": (None, [P, P, I64]),
            "orc_saug": (None, [P, I, I, I, P]),
            "orc_acf": (None, [P, I, I, P]),
            "orc_tsubcf": (None, [P, P, I, I, P]),
            "orc_im2col_cf": (None, [P, I, I, I, I, I, I, P]),
            "orc_bilinear_gather": (None, [P, I, I, I, P, I64, I, I, P]),
            "orc_gather_taps": (None, [I, I, P, I64, I, P, P, P, P]),
            "orc_bias_lrelu": (None, [P, P, I64, I, I64, I, F, P]),
            "orc_subpix_lrelu": (None, [P, P, P, I, I, I, F, P]),
            "orc_subpix_lrelu_cl": (None, [P, P, I, I, I, I, F, P]),
            "orc_upfirdn2x": (None, [P, P, I, I, I64, P]),
            "orc_clsp": (None, [P, P, P, I, I64, P]),
            "orc_flow_grid": (None, [P, P, I64, P]),
            "orc_tanh": (None, [P, I64, P]),
            "orc_sigmoid": (None, [P, I64, P]),
            "orc_conv2d_direct": (None, [P, I, I, I, P, I, I, I, I, P]),
            "orc_conv2d_s": (None, [P, I, I, I, P, I, I, I, I, I, P]),
            "orc_num_threads": (I, []),
            "orc_set_num_threads": (None, [I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def round_f16(x):
    """IEEE binary16 round-to-nearest-even, returned as f32 values."""
    y = _f32(x).copy()
    lib().orc_round_f16(_p(y), y.size)
    return y


def f16_bits(x):
    x = _f32(x)
    h = np.empty(x.shape, np.uint16)
    lib().orc_to_f16_bits(_p(x), _p(h), x.size)
    return h


def leaky(v):
    v = _f32(v)
    return np.where(v > 0, v, np.float32(SLOPE) * v).astype(np.float32, copy=False)


def bilinear_gather(feat, grid, W, H, planar=False, sp=False):
    """GGML_OP_BILINEAR_GATHER (patch :314-369). feat (W*H, C) channel-fastest;
    grid (N, 2) interleaved or (2, N) planar; returns (N, C) or (C, N) if sp."""
    feat = _f32(feat)
    grid = _f32(grid)
    C = feat.shape[-1]
    assert feat.size == C * W * H
    N = grid.size // 2
    out = np.empty((C, N) if sp else (N, C), np.float32)
    lib().orc_bilinear_gather(_p(feat), C, W, H, _p(grid), N, int(planar), int(sp), _p(out))
    return out


def gather_taps(grid, W, H, planar=False):
    grid = _f32(grid)
    N = grid.size // 2
    x0 = np.empty(N, np.int32)
    y0 = np.empty(N, np.int32)
    wx = np.empty(N, np.float32)
    wy = np.empty(N, np.float32)
    lib().orc_gather_taps(W, H, _p(grid), N, int(planar), _p(x0), _p(y0), _p(wx), _p(wy))
    return x0, y0, wx, wy


def bias_lrelu(x, b, axis, slope=SLOPE):
    """GGML_OP_BIAS_LRELU (patch :372-430). axis 0: bias over the last numpy
    dim (CL); axis 2: bias over numpy dim -3 (SP planes)."""
    x = _f32(x)
    b = _f32(b).reshape(-1)
    C = b.size
    y = np.empty_like(x)
    d01 = x.shape[-1] * x.shape[-2] if x.ndim >= 2 else 1
    lib().orc_bias_lrelu(_p(x), _p(b), x.size, C, d01, axis, slope, _p(y))
    return y


def subpix_lrelu(g0, g1, b, slope=SLOPE):
    """GGML_OP_SUBPIX_LRELU (patch :432-482): g0/g1 (2*OC, H, W) -> (OC, 2H, 2W)."""
    g0, g1, b = _f32(g0), _f32(g1), _f32(b).reshape(-1)
    C2, H, W = g0.shape
    OC = C2 // 2
    y = np.empty((OC, 2 * H, 2 * W), np.float32)
    lib().orc_subpix_lrelu(_p(g0), _p(g1), _p(b), W, H, OC, slope, _p(y))
    return y


def subpix_lrelu_cl(y4, b, W, H, slope=SLOPE):
    """GGML_OP_SUBPIX_LRELU_CL (patch :485-530): y4 (nb, W*H, 4*OC) ->
    (nb, 4*W*H, OC)."""
    y4, b = _f32(y4), _f32(b).reshape(-1)
    nb, N, OC4 = y4.shape
    OC = OC4 // 4
    assert N == W * H
    y = np.empty((nb, 4 * N, OC), np.float32)
    lib().orc_subpix_lrelu_cl(_p(y4), _p(b), OC, W, H, nb, slope, _p(y))
    return y


def upfirdn2x(x, k4):
    """GGML_OP_UPFIRDN2X (patch :532-572): x (..., H, W) -> (..., 2H, 2W)."""
    x, k4 = _f32(x), _f32(k4).reshape(-1)
    assert k4.size == 16
    H, W = x.shape[-2:]
    CB = x.size // (H * W)
    y = np.empty(x.shape[:-2] + (2 * H, 2 * W), np.float32)
    lib().orc_upfirdn2x(_p(x), _p(k4), W, H, CB, _p(y))
    return y


def clsp(cl, m, out_sp=None):
    """GGML_OP_CLSP_MUL / _LERP (patch :575-626): cl (N, C), m (N,) ->
    (C, N); lerp blends with out_sp (C, N)."""
    cl, m = _f32(cl), _f32(m).reshape(-1)
    N, C = cl.shape
    y = np.empty((C, N), np.float32)
    o = _f32(out_sp) if out_sp is not None else None
    lib().orc_clsp(_p(cl), _p(m), _p(o) if o is not None else None, C, N, _p(y))
    return y


def flow_grid(fl, xs):
    """GGML_OP_FLOW_GRID (patch :629-657): fl (3, H, W), xs (2, N) planar ->
    (3, N) planar (gx, gy, mask)."""
    fl, xs = _f32(fl), _f32(xs)
    N = fl.size // 3
    y = np.empty((3, N), np.float32)
    lib().orc_flow_grid(_p(fl), _p(xs), N, _p(y))
    return y


def tanh(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_tanh(_p(x), x.size, _p(y))
    return y


def sigmoid(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_sigmoid(_p(x), x.size, _p(y))
    return y


def im2col_cf(x_cl, W, H, round16=False):
    """channels-first im2col (patch :201-307), 3x3 stride 1 pad 1:
    x_cl (nb, W*H, IC) -> (nb, W*H, 9*IC), row r = ic + IC*(kw + 3*kh)."""
    x_cl = _f32(x_cl)
    nb, N, IC = x_cl.shape
    assert N == W * H
    out = np.empty((nb, N, 9 * IC), np.float32)
    lib().orc_im2col_cf(_p(x_cl), IC, W, H, nb, 1, int(round16), _p(out))
    return out


def conv2d_direct(x, w, pad):
    """ggml_conv_2d_direct semantics: x (IC, H, W), w (OC, IC, KH, KW)."""
    x, w = _f32(x), _f32(w)
    IC, IH, IW = x.shape
    OC, IC2, KH, KW = w.shape
    assert IC == IC2
    OH, OW = IH + 2 * pad - KH + 1, IW + 2 * pad - KW + 1
    y = np.empty((OC, OH, OW), np.float32)
    lib().orc_conv2d_direct(_p(x), IC, IH, IW, _p(w), OC, KH, KW, pad, _p(y))
    return y


def conv2d_s(x, w, stride, pad):
    """strided cross-correlation: x (IC, H, W), w (OC, IC, KH, KW)."""
    x, w = _f32(x), _f32(w)
    IC, IH, IW = x.shape
    OC, IC2, KH, KW = w.shape
    assert IC == IC2
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    y = np.empty((OC, OH, OW), np.float32)
    lib().orc_conv2d_s(_p(x), IC, IH, IW, _p(w), OC, KH, KW, stride, pad, _p(y))
    return y


def mul_mat(a, b):
    """ggml_mul_mat(a [K, M], b [K, N]) -> [M, N]; numpy a (..., M, K),
    b (..., N, K) -> (..., N, M), f32 accumulation."""
    return np.matmul(_f32(b), np.swapaxes(_f32(a), -1, -2)).astype(np.float32, copy=False)


def set_threads(n):
    lib().orc_set_num_threads(int(n))


# --------------------------------------------------------------------------
# weights: names, load-time scale folding, f16 storage rule

def weight_names(ic=REF_IC, oc=REF_OC):
    """(name, torch shape) of every decoder tensor (GGUF names)."""
    c0 = ic[0]
    v = [("dec.input.input", (1, c0, 4, 4)),
         ("dec.conv1.conv.weight", (1, c0, c0, 3, 3)),
         ("dec.conv1.conv.modulation.weight", (c0, STYLE_DIM)),
         ("dec.conv1.conv.modulation.bias", (c0,)),
         ("dec.conv1.activate.bias", (c0,))]
    for j in range(len(ic)):
        for i, (cin, cout) in ((2 * j, (ic[j], oc[j])), (2 * j + 1, (oc[j], oc[j]))):
            b = f"dec.convs.{i}"
            v += [(f"{b}.conv.weight", (1, cout, cin, 3, 3)),
                  (f"{b}.conv.modulation.weight", (cin, STYLE_DIM)),
                  (f"{b}.conv.modulation.bias", (cin,)),
                  (f"{b}.activate.bias", (cout,))]
            if i % 2 == 0:
                v.append((f"{b}.conv.blur.kernel", (4, 4)))
        f = f"dec.to_flows.{j}"
        v += [(f"{f}.conv.weight", (1, 3, oc[j], 1, 1)),
              (f"{f}.conv.modulation.weight", (oc[j], STYLE_DIM)),
              (f"{f}.conv.modulation.bias", (oc[j],)),
              (f"{f}.bias", (1, 3, 1, 1)),
              (f"{f}.upsample.kernel", (4, 4))]
        r = f"dec.to_rgbs.{j}"
        v += [(f"{r}.conv.0.weight", (3, oc[j], 1, 1)),
              (f"{r}.conv.1.bias", (3,)),
              (f"{r}.bias", (1, 3, 1, 1)),
              (f"{r}.upsample.kernel", (4, 4))]
    return v


def ggml_ne(shape):
    """ggml ne of a torch shape after the loader drops leading unit dims only
    where they do not fit (src/gguf_load.cpp:111-124): reversed order."""
    ne = list(reversed(shape))
    while len(ne) > 4 and ne[-1] == 1:
        ne.pop()
    return ne + [1] * (4 - len(ne))


def motion_ae_scale(name, ne):
    """Load-time scale folding (src/motion_enc.cpp:14-45), decoder subset."""
    if (name.endswith(".activate.bias") or
            (name.startswith("dec.to_rgbs.") and name.endswith(".conv.1.bias"))):
        return SQRT2
    if not name.endswith(".weight"):
        return 1.0
    if name.startswith("dec.direction") or name.endswith("noise.weight"):
        return 1.0
    if name.endswith("modulation.weight"):
        return 1.0 / math.sqrt(float(ne[0]))
    conv = 1.0 / math.sqrt(float(ne[0] * ne[1] * ne[2]))
    if name.startswith("dec.to_rgbs.") and name.endswith(".conv.0.weight"):
        return conv * SQRT2
    if name.endswith(".conv.weight"):
        return conv
    return 1.0


def load_weights(raw, keep_f16):
    """Restates weights_t::load's numeric path (src/gguf_load.cpp:146-194):
    raw[name] = (array in torch shape, f16_in_file).  Returns
      dev[name]  : values as the device tensor holds them (f16-rounded when
                   kept f16: file-f16 AND >= 4096 elements)
      host[name] : scale-folded f32 host copy (before any f16 storage
                   rounding) — what prepare() reads
      isf16[name]: whether the device tensor is F16."""
    dev, host, isf16 = {}, {}, {}
    for name, (arr, f16_in_file) in raw.items():
        a = _f32(arr)
        if f16_in_file:
            a = round_f16(a)  # the file holds f16 values
        s = motion_ae_scale(name, ggml_ne(a.shape))
        if s != 1.0:
            a = (a * np.float32(s)).astype(np.float32, copy=False)
        host[name] = a
        big = keep_f16 and f16_in_file and a.size >= 4096
        isf16[name] = big
        dev[name] = round_f16(a) if big else a
    return dev, host, isf16


# --------------------------------------------------------------------------
# the decoder

class Decoder:
    """Oracle decoder over a full set of raw weights (see load_weights).

    ic/oc: per-stage channel lists (the reference's REF_IC/REF_OC; smaller
    lists give the same graph with fewer channels, for fast tests)."""

    def __init__(self, raw, ftype="f32", ic=REF_IC, oc=REF_OC):
        assert ftype in ("f32", "f16")
        assert len(ic) == len(oc) and all(ic[j + 1] == oc[j] for j in range(len(ic) - 1))
        self.f16 = ftype == "f16"
        self.ic, self.oc = tuple(ic), tuple(oc)
        self.n_stages = len(ic)
        self.w, self.host, self.isf16 = load_weights(raw, self.f16)
        self.prepare()
        self.feats = None

    # ---- prepare (src/motion_dec.cpp:31-226)
    def prepare(self):
        L = lib()
        self.der = {}
        jobs = [("dec.conv1.conv.weight", self.ic[0], self.ic[0], False)]
        for j in range(self.n_stages):
            jobs.append((f"dec.convs.{2 * j}.conv.weight", self.ic[j], self.oc[j], True))
            jobs.append((f"dec.convs.{2 * j + 1}.conv.weight", self.oc[j], self.oc[j], False))
        for name, IC, OC, flip in jobs:
            if name not in self.host:
                raise KeyError("host copy missing for " + name)
            W = _f32(self.host[name].reshape(OC, IC, 3, 3))
            sa = np.empty((OC, IC + 1), np.float32)
            L.orc_saug(_p(W), OC, IC, 9, _p(sa))
            self.der["saug." + name] = sa
            wt = round_f16 if self.f16 else (lambda a: a)
            if not flip and name != "dec.conv1.conv.weight":
                ac = np.empty((OC, 9 * IC), np.float32)
                L.orc_acf(_p(W), OC, IC, _p(ac))
                self.der["acf." + name] = wt(ac)
            if flip:
                bk_name = name[: -len("weight")] + "blur.kernel"
                BK = _f32(self.host[bk_name]).reshape(16)
                ts = np.empty((4 * OC, 9 * IC), np.float32)
                L.orc_tsubcf(_p(W), _p(BK), OC, IC, _p(ts))
                self.der["tsubcf." + name] = wt(ts)
                # spatial layout [4OC][IC][kh][kw] of the same values
                tsp = ts.reshape(4 * OC, 3, 3, IC).transpose(0, 3, 1, 2)
                self.der["tsubsp." + name] = wt(np.ascontiguousarray(tsp))
                self.der["wflip." + name] = np.ascontiguousarray(W[:, :, ::-1, ::-1])

    def set_feats(self, feats):
        """feats[j]: (r_j*r_j, OC_j) pixel-major, channel fastest
        (src/motion_dec.cpp:1137-1160); f16-rounded in f16 mode."""
        assert len(feats) == self.n_stages
        out = []
        for j, f in enumerate(feats):
            r = 8 << j
            f = _f32(f).reshape(r * r, self.oc[j])
            out.append(round_f16(f) if self.f16 else f)
        self.feats = out

    # ---- per-frame style vectors
    def style_of(self, base, latent):
        """linear(mw, mb, latent) (src/motion_dec.cpp:267-272):
        latent (B, 512) -> (B, IC)."""
        mw = self.w[base + ".modulation.weight"]
        mb = self.w[base + ".modulation.bias"].reshape(-1)
        return (mul_mat(mw, latent) + mb).astype(np.float32, copy=False)

    def demod_den(self, wname, s):
        """sqrt(S_aug . [s^2; 1]) (src/motion_dec.cpp:275-280): (B, OC)."""
        sa = self.der["saug." + wname]
        s2 = np.concatenate([_f32(s) * _f32(s), np.ones((s.shape[0], 1), np.float32)], axis=1)
        return np.sqrt(mul_mat(sa, s2)).astype(np.float32, copy=False)

    @staticmethod
    def lin(r):
        i = np.arange(r, dtype=np.float64)
        return (-1.0 + 2.0 * i / (r - 1)).astype(np.float32, copy=False)

    # ------------------------------------------------------------------
    # exact (parity) graph, one frame, f32 (src/motion_dec.cpp:794-888)

    def _styled_conv_exact(self, x, base, latent):
        s = self.style_of(base + ".conv", latent[None])[0]
        den = self.demod_den(base + ".conv.weight", s[None])[0]
        W = self.w[base + ".conv.weight"].reshape(den.size, s.size, 3, 3)
        ab = self.w[base + ".activate.bias"].reshape(-1)
        xs = (x * s[:, None, None]).astype(np.float32, copy=False)
        y = conv2d_direct(xs, W, 1)
        y = (y / den[:, None, None]).astype(np.float32, copy=False)
        return leaky(y + ab[:, None, None])

    def _styled_conv_up_exact(self, x, base, latent):
        s = self.style_of(base + ".conv", latent[None])[0]
        den = self.demod_den(base + ".conv.weight", s[None])[0]
        Wf = self.der["wflip." + base + ".conv.weight"]
        kb = self.w[base + ".conv.blur.kernel"].reshape(4, 4)
        ab = self.w[base + ".activate.bias"].reshape(-1)
        C, H, W = x.shape
        xs = (x * s[:, None, None]).astype(np.float32, copy=False)
        zs = np.zeros((C, 2 * H + 3, 2 * W + 3), np.float32)   # zero_stuff2 + pad(2,1)
        zs[:, 2:2 * H + 2:2, 2:2 * W + 2:2] = xs
        y = conv2d_direct(zs, Wf, 0)                           # (OC, 2H+1, 2W+1)
        y = (y / den[:, None, None]).astype(np.float32, copy=False)
        OC = y.shape[0]
        yp = np.zeros((OC, 2 * H + 3, 2 * W + 3), np.float32)  # blur pad (1,1)
        yp[:, 1:-1, 1:-1] = y
        # depthwise 4x4 cross-correlation, per channel (ggml_conv_2d_dw_direct)
        yb = np.zeros((OC, 2 * H, 2 * W), np.float32)
        for kh in range(4):
            for kw in range(4):
                yb += np.float32(kb[kh, kw]) * yp[:, kh:kh + 2 * H, kw:kw + 2 * W]
        return leaky(yb + ab[:, None, None])

    def decode_exact(self, latent, n_stages=None):
        """One frame: latent (512,) -> (img (3, R, R), taps dict).  Tap names
        follow src/motion_dec.cpp:805-883."""
        assert not self.f16, "the exact graph oracle is f32"
        latent = _f32(latent).reshape(STYLE_DIM)
        ns = self.n_stages if n_stages is None else n_stages
        taps = {}
        cinp = self.w["dec.input.input"].reshape(self.ic[0], 4, 4)
        out = self._styled_conv_exact(cinp, "dec.conv1", latent)
        taps["conv1_4"] = out
        skip = skip_flow = None
        for j in range(ns):
            r = 8 << j
            out = self._styled_conv_up_exact(out, f"dec.convs.{2 * j}", latent)
            taps[f"r{r}.conv1"] = out
            out = self._styled_conv_exact(out, f"dec.convs.{2 * j + 1}", latent)
            taps[f"r{r}.conv2"] = out
            fb = f"dec.to_flows.{j}"
            fs = self.style_of(fb + ".conv", latent[None])[0]
            fW = self.w[fb + ".conv.weight"].reshape(3, -1, 1, 1)
            xs = (out * fs[:, None, None]).astype(np.float32, copy=False)
            fl = conv2d_direct(xs, fW, 0) + self.w[fb + ".bias"].reshape(3, 1, 1)
            fl = fl.astype(np.float32, copy=False)
            if skip_flow is not None:
                fl = (fl + upfirdn2x(skip_flow, self.w[fb + ".upsample.kernel"])).astype(np.float32, copy=False)
            skip_flow = fl
            taps[f"r{r}.flowmap"] = fl
            lin = self.lin(r)
            gx = (tanh(fl[0]) + lin[None, :]).astype(np.float32, copy=False)
            gy = (tanh(fl[1]) + lin[:, None]).astype(np.float32, copy=False)
            taps[f"r{r}.grid"] = np.stack([gx, gy], axis=-1)
            m = sigmoid(fl[2])
            grid = np.stack([gx.reshape(-1), gy.reshape(-1)], axis=1)
            sampled = bilinear_gather(self.feats[j], grid, r, r)        # (N, C)
            sampled = np.ascontiguousarray(sampled.T.reshape(-1, r, r))  # cl_to_sp
            warp = (sampled * m[None]).astype(np.float32, copy=False)
            taps[f"r{r}.warp"] = warp
            one_m = (np.float32(1.0) - m).astype(np.float32, copy=False)
            trunk = (warp + (out * one_m[None]).astype(np.float32, copy=False)).astype(np.float32, copy=False)
            taps[f"r{r}.out"] = trunk
            rb = f"dec.to_rgbs.{j}"
            rW = self.w[rb + ".conv.0.weight"].reshape(3, -1, 1, 1)
            rgb = conv2d_direct(warp, rW, 0)
            rgb = leaky(rgb + self.w[rb + ".conv.1.bias"].reshape(3, 1, 1))
            rgb = (rgb + self.w[rb + ".bias"].reshape(3, 1, 1)).astype(np.float32, copy=False)
            if skip is not None:
                rgb = (rgb + upfirdn2x(skip, self.w[rb + ".upsample.kernel"])).astype(np.float32, copy=False)
            skip = rgb
            taps[f"r{r}.rgb"] = rgb
            out = trunk
        return skip, taps

    # ------------------------------------------------------------------
    # fast channel-last graph (src/motion_dec.cpp:889-1123)

    @staticmethod
    def fold_into_weights(wsz, N, ic, oc):
        """src/motion_dec.cpp:318-320"""
        return 4 * wsz < 2 * N * (ic + oc)

    def _r16(self, a):
        return round_f16(a) if self.f16 else _f32(a)

    def _fold_A(self, A, s, den):
        """fold_A (src/motion_dec.cpp:323-337): A (M, R) -> (B, M, R) with
        A * s[r % IC] / den[q]; cast back to the weight dtype."""
        Bc = s.shape[0]
        IC = s.shape[1]
        R = A.shape[1]
        sty = np.tile(s, (1, R // IC))                       # (B, R)
        Af = (A[None] * sty[:, None, :]).astype(np.float32, copy=False)
        Af = (Af / den[:, :, None]).astype(np.float32, copy=False)
        return self._r16(Af)

    def _conv_cf(self, A, Af, x_cl, W, H, round_in):
        """conv_cf (src/motion_dec.cpp:340-354): x_cl (B, W*H, IC) ->
        (B, W*H, M).  Af is A itself (shared) or folded (B, M, R)."""
        im = im2col_cf(x_cl, W, H, round16=round_in)
        if Af is A:
            return mul_mat(A, im)
        return mul_mat(Af, im)

    def _styled_conv_up_cl(self, x_cl, W, H, base, s, den):
        """styled_conv_up + subpix_lrelu_cl (src/motion_dec.cpp:397-433)."""
        Ts = self.der["tsubcf." + base + ".conv.weight"]
        ab = self.w[base + ".activate.bias"]
        OC4, R = Ts.shape
        IC = x_cl.shape[2]
        N = W * H
        den4 = np.tile(den, (1, 4))                           # q % OC = o
        if self.fold_into_weights(R * OC4, N, IC, OC4):
            y4 = self._conv_cf(Ts, self._fold_A(Ts, s, den4), x_cl, W, H, self.f16)
        else:
            xs = (x_cl * s[:, None, :]).astype(np.float32, copy=False)
            y4 = self._conv_cf(Ts, Ts, xs, W, H, self.f16)
            y4 = (y4 / den4[:, None, :]).astype(np.float32, copy=False)
        return subpix_lrelu_cl(y4, ab, W, H)

    def _styled_conv_cl(self, x_cl, W, H, base, s, den):
        """styled_conv (src/motion_dec.cpp:357-373)."""
        A = self.der["acf." + base + ".conv.weight"]
        ab = self.w[base + ".activate.bias"]
        OC, R = A.shape
        IC = x_cl.shape[2]
        if self.fold_into_weights(R * OC, W * H, IC, OC):
            y = self._conv_cf(A, self._fold_A(A, s, den), x_cl, W, H, self.f16)
        else:
            xs = (x_cl * s[:, None, :]).astype(np.float32, copy=False)
            y = self._conv_cf(A, A, xs, W, H, self.f16)
            y = (y / den[:, None, :]).astype(np.float32, copy=False)
        return bias_lrelu(y, ab, 0)

    def _conv1(self, s0, d0):
        """styled_conv_input (src/motion_dec.cpp:375-393): (B, 16, C0)."""
        C0 = self.ic[0]
        x = self.w["dec.input.input"].reshape(C0, 4, 4)
        Bb = s0.shape[0]
        xs = (x[None] * s0[:, :, None, None]).astype(np.float32, copy=False)   # (B, C0, 4, 4)
        if self.isf16["dec.input.input"]:
            xs = round_f16(xs)  # F16 tensor result of ggml_mul
        W = self.w["dec.conv1.conv.weight"].reshape(C0, C0 * 9)      # row kw + 3kh + 9ic
        # stock im2col: rows ic*9 + kh*3 + kw over the SP map
        pad = np.zeros((Bb, C0, 6, 6), np.float32)
        pad[:, :, 1:5, 1:5] = xs
        im = np.empty((Bb, 16, C0 * 9), np.float32)
        for oy in range(4):
            for ox in range(4):
                im[:, oy * 4 + ox, :] = pad[:, :, oy:oy + 3, ox:ox + 3].reshape(Bb, -1)
        y = mul_mat(W, self._r16(im) if self.f16 else im)              # (B, 16, C0)
        y = (y / d0[:, None, :]).astype(np.float32, copy=False)
        return bias_lrelu(y, self.w["dec.conv1.activate.bias"], 0)

    def _fold_w4(self, W4, s, den):
        """fold_w4 (src/motion_dec.cpp:451-465) on torch-order weights
        (OC', IC, kh, kw), one frame: W * s[ic] / den[oc'] -> weight dtype."""
        Wf = _f32(W4)
        if s is not None:
            Wf = (Wf * s[None, :, None, None]).astype(np.float32, copy=False)
        if den is not None:
            Wf = (Wf / den[:, None, None, None]).astype(np.float32, copy=False)
        return Wf

    def _conv_sp(self, x_sp, Wt, round_in):
        """ggml_conv_2d_direct 3x3 pad 1 on one SP frame (C, H, W) via the
        cf-im2col + GEMM route: (OC', H, W)."""
        C, H, W = x_sp.shape
        x_cl = np.ascontiguousarray(x_sp.transpose(1, 2, 0).reshape(1, H * W, C))
        im = im2col_cf(x_cl, W, H, round16=round_in)
        A = np.ascontiguousarray(Wt.transpose(0, 2, 3, 1).reshape(Wt.shape[0], -1))
        y = mul_mat(A, im)[0]                                          # (H*W, OC')
        return np.ascontiguousarray(y.T.reshape(-1, H, W))

    def tail_cl(self, j, out, fs, skf, sk):
        """channel-last stage tail (src/motion_dec.cpp:1077-1108): out (B, N, C),
        ToFlow style fs (B, C), previous flow/rgb skips (B, 3, r/2, r/2) or None
        -> flowmap (B, 3, r, r), warp (B, N, C), trunk (B, N, C), rgb (B, 3, r, r)"""
        r = 8 << j
        Bb, N, C = out.shape
        fb, rb = f"dec.to_flows.{j}", f"dec.to_rgbs.{j}"
        fW = self.w[fb + ".conv.weight"].reshape(3, -1)
        fbias = self.w[fb + ".bias"].reshape(3)
        rW = self.w[rb + ".conv.0.weight"].reshape(3, -1)
        rlb = self.w[rb + ".conv.1.bias"].reshape(3)
        rbias = self.w[rb + ".bias"].reshape(3)
        lin = self.lin(r)
        # ToFlow: gemm_weight(fW, fstyle) then mul_mat (:1077-1085)
        Af = (fW[None] * fs[:, None, :]).astype(np.float32, copy=False)            # (B, 3, C)
        fl_cl = mul_mat(Af, out)                                        # (B, N, 3)
        fl_cl = (fl_cl + fbias).astype(np.float32, copy=False)
        fl = np.ascontiguousarray(fl_cl.transpose(0, 2, 1).reshape(Bb, 3, r, r))
        if skf is not None:
            fl = (fl + upfirdn2x(skf, self.w[fb + ".upsample.kernel"])).astype(np.float32, copy=False)
        gx = (tanh(fl[:, 0]) + lin[None, None, :]).astype(np.float32, copy=False)
        gy = (tanh(fl[:, 1]) + lin[None, :, None]).astype(np.float32, copy=False)
        m = sigmoid(fl[:, 2])                                           # (B, r, r)
        grid = np.stack([gx.reshape(-1), gy.reshape(-1)], axis=1)       # [2, N*B]
        sampled = bilinear_gather(self.feats[j], grid, r, r).reshape(Bb, N, C)
        m_row = m.reshape(Bb, N, 1)
        warp = (sampled * m_row).astype(np.float32, copy=False)
        one_m = (np.float32(1.0) - m_row).astype(np.float32, copy=False)
        trunk = (warp + (out * one_m).astype(np.float32, copy=False)).astype(np.float32, copy=False)
        rgb_cl = mul_mat(rW, warp)                                      # (B, N, 3)
        rgb_cl = bias_lrelu(rgb_cl, rlb, 0)
        rgb_cl = (rgb_cl + rbias).astype(np.float32, copy=False)
        rgb = np.ascontiguousarray(rgb_cl.transpose(0, 2, 1).reshape(Bb, 3, r, r))
        if sk is not None:
            rgb = (rgb + upfirdn2x(sk, self.w[rb + ".upsample.kernel"])).astype(np.float32, copy=False)
        return fl, warp, trunk, rgb

    def decode_fast(self, latents, n_stages=None, want_taps=False):
        """Batched fast graph: latents (B, 512) -> imgs (B, 3, R, R) f32 [and
        per-stage taps: c1, out, flowmap, warp, trunk, rgb per frame]."""
        lat = _f32(latents).reshape(-1, STYLE_DIM)
        Bb = lat.shape[0]
        ns = self.n_stages if n_stages is None else n_stages
        spatial_from = 5
        taps = {}
        s0 = self.style_of("dec.conv1.conv", lat)
        d0 = self.demod_den("dec.conv1.conv.weight", s0)
        x = self._conv1(s0, d0)                # CL (B, 16, C0)
        x_is_sp = False
        if want_taps:
            taps["conv1_4"] = x
        sk = skf = None                        # SP (B, 3, r, r)
        for j in range(ns):
            r = 8 << j
            N = r * r
            b1, b2 = f"dec.convs.{2 * j}", f"dec.convs.{2 * j + 1}"
            fb, rb = f"dec.to_flows.{j}", f"dec.to_rgbs.{j}"
            s1 = self.style_of(b1 + ".conv", lat)
            d1 = self.demod_den(b1 + ".conv.weight", s1)
            s2 = self.style_of(b2 + ".conv", lat)
            d2 = self.demod_den(b2 + ".conv.weight", s2)
            fs = self.style_of(fb + ".conv", lat)
            fW = self.w[fb + ".conv.weight"].reshape(3, -1)
            fbias = self.w[fb + ".bias"].reshape(3)
            fup = self.w[fb + ".upsample.kernel"]
            rW = self.w[rb + ".conv.0.weight"].reshape(3, -1)
            rlb = self.w[rb + ".conv.1.bias"].reshape(3)
            rbias = self.w[rb + ".bias"].reshape(3)
            rup = self.w[rb + ".upsample.kernel"]
            C = self.oc[j]
            lin = self.lin(r)
            if j >= spatial_from:
                xn, skn, sfn = [], [], []
                tc1, tout, twarp = [], [], []
                for c in range(Bb):
                    if x_is_sp:
                        x_c = x[c]
                    else:  # cl_to_sp
                        x_c = np.ascontiguousarray(x[c].reshape(r // 2, r // 2, -1).transpose(2, 0, 1))
                    # styled_conv_up_sp (:479-594): folded composed kernel,
                    # 4 classes on the channel dim, subpix_lrelu
                    Ts = self.der["tsubsp." + b1 + ".conv.weight"]
                    den4 = np.tile(d1[c], 4)
                    Wf = self._r16(self._fold_w4(Ts, s1[c], den4))
                    y4 = self._conv_sp(x_c, Wf, self.f16)             # (4OC, r/2, r/2)
                    c1 = subpix_lrelu(y4[:2 * C], y4[2 * C:], self.w[b1 + ".activate.bias"])
                    # styled_conv_sp (:467-475)
                    W2 = self.w[b2 + ".conv.weight"].reshape(C, C, 3, 3)
                    W2f = self._r16(self._fold_w4(W2, s2[c], d2[c]))
                    y = self._conv_sp(c1, W2f, self.f16)
                    out = bias_lrelu(y, self.w[b2 + ".activate.bias"], 2)
                    # ToFlow 1x1, weight-folded f32
                    fWf = (fW * fs[c][None, :]).astype(np.float32, copy=False)
                    fl = mul_mat(fWf, np.ascontiguousarray(out.reshape(C, -1).T)).T.reshape(3, r, r)
                    fl = (fl + fbias[:, None, None]).astype(np.float32, copy=False)
                    if skf is not None:
                        fl = (fl + upfirdn2x(skf[c], fup)).astype(np.float32, copy=False)
                    sfn.append(fl)
                    xsg = np.stack([np.tile(lin, r), np.repeat(lin, r)])     # (2, N) planar
                    fg = flow_grid(fl, xsg)
                    sampled = bilinear_gather(self.feats[j], np.ascontiguousarray(fg[:2]),
                                              r, r, planar=True)             # (N, C)
                    m = fg[2]
                    warp = clsp(sampled, m).reshape(C, r, r)
                    trunk = clsp(sampled, m, out.reshape(C, N)).reshape(C, r, r)
                    xn.append(trunk)
                    rgb = mul_mat(rW, np.ascontiguousarray(warp.reshape(C, -1).T)).T.reshape(3, r, r)
                    rgb = bias_lrelu(np.ascontiguousarray(rgb), rlb, 2)
                    rgb = (rgb + rbias[:, None, None]).astype(np.float32, copy=False)
                    if sk is not None:
                        rgb = (rgb + upfirdn2x(sk[c], rup)).astype(np.float32, copy=False)
                    skn.append(rgb)
                    if want_taps:
                        tc1.append(c1)
                        tout.append(out)
                        twarp.append(warp)
                x, sk, skf = np.stack(xn), np.stack(skn), np.stack(sfn)
                x_is_sp = True
                if want_taps:
                    taps[f"r{r}.conv1"] = np.stack(tc1)      # SP (B, C, r, r)
                    taps[f"r{r}.conv2"] = np.stack(tout)
                    taps[f"r{r}.flowmap"] = skf
                    taps[f"r{r}.warp"] = np.stack(twarp)
                    taps[f"r{r}.out"] = x
                    taps[f"r{r}.rgb"] = sk
                continue
            # ---- channel-last stage
            c1 = self._styled_conv_up_cl(x, r // 2, r // 2, b1, s1, d1)    # (B, N, C)
            out = self._styled_conv_cl(c1, r, r, b2, s2, d2)
            fl, warp, trunk, rgb = self.tail_cl(j, out, fs, skf, sk)
            if want_taps:
                taps[f"r{r}.conv1"] = c1
                taps[f"r{r}.conv2"] = out
                taps[f"r{r}.flowmap"] = fl
                taps[f"r{r}.warp"] = warp
                taps[f"r{r}.out"] = trunk
                taps[f"r{r}.rgb"] = rgb
            x, sk, skf = trunk, rgb, fl
        return (sk, taps) if want_taps else sk
