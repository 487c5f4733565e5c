"""Stage-by-stage oracle check of the decode chain as decode_batch runs it.

The decoder's taps (tpmd_set_tap) copy the buffers its launches pass to one
another: conv1's output, each up-conv's output (c1), each stage's trunk,
flow map and rgb skip, and the dense-conv output of the stages whose tail
runs in a kernel of its own.  Each launch group is checked against the CPU
oracle fed the GPU's own input to that group, so every stage is graded on
its own and no rounding difference is carried (and, through the warp,
amplified) from one stage into the next:

  conv1        oracle conv1 (styled_conv_input) x the stage-0 up-conv style
  up-conv j    oracle sub-pixel GEMM of the GPU's trunk (j-1), x the dense
               conv's style, rounded to the activation type
  dense conv j oracle styled conv of the GPU's c1 (j); its output feeds
  tail j       the oracle's stage tail with the GPU's flow/rgb skips (j-1):
               the flow map is compared directly; the warp and everything
               built on it (trunk, rgb, the frame) are compared against the
               oracle's gather driven by the GPU's own flow map, because the
               bilinear warp moves a flow difference d by about d * r / 2
               pixels (a rounding-level conv difference would otherwise
               decide the comparison at r512 on i.i.d. inputs)

Tolerances: f32 rel-L2 <= 1e-4; f16 rel-L2 <= 1e-2 and cosine >= 0.9999."""
import numpy as np

import tpmd
from metrics import cosine, rel_l2

KINDS = (tpmd.TAP_TRUNK, tpmd.TAP_C1, tpmd.TAP_OUT, tpmd.TAP_FLOW, tpmd.TAP_RGB)


def register_taps(torch, dec, n):
    """a device buffer for every tap the chain holds; {(kind, stage): tensor}"""
    act = torch.float16 if dec.ftype == "f16" else torch.float32
    bufs = {}
    for kind in KINDS:
        for stage in range(-1, dec.n_stages):
            fb = dec.tap_frame_bytes(kind, stage)
            if fb < 0:
                continue
            dt = act if kind in (tpmd.TAP_TRUNK, tpmd.TAP_C1) else torch.float32
            t = torch.empty((n, fb // (2 if dt == torch.float16 else 4)), dtype=dt, device="cuda")
            dec.set_tap(kind, stage, t)
            bufs[(kind, stage)] = t
    return bufs


def clear_taps(dec, bufs):
    for kind, stage in bufs:
        dec.set_tap(kind, stage, None)


def frames_of(bufs, kind, stage, F):
    """frames F of a tap as f32 numpy, (len(F), per-frame elements)"""
    import torch
    t = bufs[(kind, stage)][torch.as_tensor(F, device="cuda")]
    return t.float().cpu().numpy()


def _check(ftype, got, want, what, report):
    e = rel_l2(got, want)
    c = cosine(got, want)
    report.append((what, e, c))
    if ftype == "f32":
        assert e <= 1e-4, (what, e)
    else:
        assert e <= 1e-2 and c >= 0.9999, (what, e, c)


def warp_from_flow(om, ref, j, fl):
    """the oracle's grid_sample warp of stage j driven by a flow map
    (n, 3, r, r): tanh / sigmoid flow head, identity grid, bilinear gather
    (src/motion_dec.cpp:1087-1097); returns warp (n, r*r, C) and the mask
    (n, r*r, 1)"""
    r = 8 << j
    nf = fl.shape[0]
    lin = ref.lin(r)
    gx = (om.tanh(fl[:, 0]) + lin[None, None, :]).astype(np.float32)
    gy = (om.tanh(fl[:, 1]) + lin[None, :, None]).astype(np.float32)
    m = om.sigmoid(fl[:, 2]).reshape(nf, r * r, 1)
    grid = np.stack([gx.reshape(-1), gy.reshape(-1)], 1)
    smp = om.bilinear_gather(ref.feats[j], grid, r, r).reshape(nf, r * r, -1)
    return (smp * m).astype(np.float32), m


def check_chain(om, ref, bufs, lat, F, imgs_F, ftype):
    """grade every launch group of the decode of latents lat[F] (frames F of
    the tapped call; imgs_F their frames); returns [(what, rel-L2, cosine)]"""
    act = om.round_f16 if ref.f16 else om._f32
    latF = lat[F]
    nf = len(F)
    report = []
    st = lambda base: ref.style_of(base + ".conv", latF)
    ns = ref.n_stages
    C0 = ref.ic[0]
    s0 = st("dec.conv1")
    s_up = st("dec.convs.0")
    x = ref._conv1(s0, ref.demod_den("dec.conv1.conv.weight", s0))            # (F, 16, C0)
    want = act(x * s_up[:, None, :])
    got = frames_of(bufs, tpmd.TAP_TRUNK, -1, F).reshape(nf, 16, C0)
    _check(ftype, got, want, "conv1", report)
    x = got
    skf = sk = None
    for j in range(ns):
        r, rh, C = 8 << j, 4 << j, ref.oc[j]
        b1, b2 = f"dec.convs.{2 * j}", f"dec.convs.{2 * j + 1}"
        fb, rb = f"dec.to_flows.{j}", f"dec.to_rgbs.{j}"
        last = j == ns - 1
        s1, s2 = st(b1), st(b2)
        d1 = ref.demod_den(b1 + ".conv.weight", s1)
        d2 = ref.demod_den(b2 + ".conv.weight", s2)
        # up-conv on the GPU's (pre-scaled) operand: map-side composed GEMM
        Ts = ref.der["tsubcf." + b1 + ".conv.weight"]
        y4 = om.mul_mat(Ts, om.im2col_cf(x, rh, rh, round16=ref.f16))
        y4 = (y4 / np.tile(d1, (1, 4))[:, None, :]).astype(np.float32)
        c1 = om.subpix_lrelu_cl(y4, ref.w[b1 + ".activate.bias"], rh, rh)      # (F, r*r, C)
        got = frames_of(bufs, tpmd.TAP_C1, j, F).reshape(nf, r * r, C)
        _check(ftype, got, act(c1 * s2[:, None, :]), (j, "up-conv"), report)
        # dense conv on the GPU's c1
        A = ref.der["acf." + b2 + ".conv.weight"]
        y = om.mul_mat(A, om.im2col_cf(got, r, r, round16=ref.f16))
        out = om.bias_lrelu((y / d2[:, None, :]).astype(np.float32), ref.w[b2 + ".activate.bias"], 0)
        if (tpmd.TAP_OUT, j) in bufs:
            _check(ftype, frames_of(bufs, tpmd.TAP_OUT, j, F).reshape(nf, r * r, C), out, (j, "conv"), report)
        fs = st(fb)
        fl, _, _, _ = ref.tail_cl(j, out, fs, skf, sk)
        gfl = frames_of(bufs, tpmd.TAP_FLOW, j, F).reshape(nf, 3, r, r)
        _check(ftype, gfl, fl, (j, "flow"), report)
        warp, m = warp_from_flow(om, ref, j, gfl)
        rW = ref.w[rb + ".conv.0.weight"].reshape(3, -1)
        rgb = om.bias_lrelu(om.mul_mat(rW, warp), ref.w[rb + ".conv.1.bias"].reshape(3), 0)
        rgb = (rgb + ref.w[rb + ".bias"].reshape(3)).astype(np.float32)
        rgb = np.ascontiguousarray(rgb.transpose(0, 2, 1).reshape(nf, 3, r, r))
        if sk is not None:
            rgb = (rgb + om.upfirdn2x(sk, ref.w[rb + ".upsample.kernel"])).astype(np.float32)
        if last:
            _check(ftype, imgs_F, rgb, (j, "frame"), report)
            break
        grgb = frames_of(bufs, tpmd.TAP_RGB, j, F).reshape(nf, 3, r, r)
        _check(ftype, grgb, rgb, (j, "rgb"), report)
        trunk = (warp + (out * (np.float32(1.0) - m)).astype(np.float32)).astype(np.float32)
        s_next = st(f"dec.convs.{2 * j + 2}")
        got = frames_of(bufs, tpmd.TAP_TRUNK, j, F).reshape(nf, r * r, C)
        _check(ftype, got, act(trunk * s_next[:, None, :]), (j, "trunk"), report)
        x, skf, sk = got, gfl, grgb
    return report
