"""Pins the CPU oracle's op restatements against independent formulations:
numpy's IEEE float16, torch-CPU library routines (grid_sample, conv2d,
conv_transpose2d, unfold), the reference's own naive upfirdn2d known-answer
check (tests/test_ops.cpp:16-106), closed forms and special cases."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from lia_torch import upfirdn2d as torch_upfirdn2d


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- f16 rounding

def test_f16_rounding_matches_numpy(om):
    g = rng(1)
    vals = [g.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 1e3, 7e4)]
    special = np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e9, np.inf, -np.inf,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 2.0 ** -14,
                        2.0 ** -14 * 0.99999, 3 * 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11,
                        1 + 2.0 ** -11 + 2.0 ** -20], np.float32)
    # every f32 bit pattern near a grid of f16 boundaries (ties and neighbours)
    h = np.arange(0, 0x7c00, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = (h[:-1].astype(np.float64) + h[1:]) / 2
    near = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
                           np.nextafter(mids.astype(np.float32), np.float32(-np.inf)),
                           mids.astype(np.float32)])
    x = np.concatenate(vals + [special, near, -near])
    got = om.round_f16(x)
    with np.errstate(over="ignore"):
        want16 = x.astype(np.float16)
    want = want16.astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(om.f16_bits(x), want16.view(np.uint16))


def test_f16_nan(om):
    got = om.round_f16(np.array([np.nan], np.float32))
    assert np.isnan(got[0])


# ---------------------------------------------------------------- gather

def torch_grid_sample(feat, W, H, grid):
    """feat (W*H, C) pixel-major; grid (N, 2) -> (N, C) via torch CPU"""
    C = feat.shape[1]
    f = torch.tensor(feat, dtype=torch.float64).reshape(H, W, C).permute(2, 0, 1)[None]
    g = torch.tensor(grid, dtype=torch.float64).reshape(1, 1, -1, 2)
    out = F.grid_sample(f, g, mode="bilinear", padding_mode="zeros", align_corners=False)
    return out[0, :, 0, :].T.numpy()


@pytest.mark.parametrize("W,H,C", [(9, 7, 16), (64, 64, 8), (1, 1, 4), (2, 5, 3)])
def test_gather_vs_torch_grid_sample(om, W, H, C):
    g = rng(W * 100 + H)
    feat = g.standard_normal((W * H, C)).astype(np.float32)
    grid = g.uniform(-1.3, 1.3, (500, 2)).astype(np.float32)
    got = om.bilinear_gather(feat, grid, W, H)
    want = torch_grid_sample(feat, W, H, grid)
    assert np.abs(got - want).max() < 2e-5 * max(1.0, np.abs(want).max())
    # planar grid and SP output are the same numbers, bit for bit
    gp = np.ascontiguousarray(grid.T)
    assert np.array_equal(om.bilinear_gather(feat, gp, W, H, planar=True), got)
    assert np.array_equal(om.bilinear_gather(feat, grid, W, H, sp=True), got.T)


def test_gather_special_cases(om):
    W, H, C = 12, 10, 5
    g = rng(7)
    feat = g.standard_normal((W * H, C)).astype(np.float32)
    # pixel centres of the map: every sample is exactly one tap (weight 1)
    xs = (2 * np.arange(W, dtype=np.float64) + 1) / W - 1
    ys = (2 * np.arange(H, dtype=np.float64) + 1) / H - 1
    gy, gx = np.meshgrid(ys, xs, indexing="ij")
    grid = np.stack([gx.ravel(), gy.ravel()], 1).astype(np.float32)
    x0, y0, wx, wy = om.gather_taps(grid, W, H)
    exact = (wx == 0) & (wy == 0)
    assert exact.mean() > 0.5  # representable centres land exactly
    got = om.bilinear_gather(feat, grid, W, H)
    idx = (y0 * W + x0)[exact]
    assert np.array_equal(got[exact], feat[idx])
    # every tap out of range -> exact zeros
    far = g.uniform(1.2, 3.0, (300, 2)).astype(np.float32) * np.where(g.random((300, 2)) < 0.5, 1, -1).astype(np.float32)
    assert np.array_equal(om.bilinear_gather(feat, far, W, H), np.zeros((300, C), np.float32))
    # the four taps: weights sum to 1, indices are floor(fx)
    grid = g.uniform(-1, 1, (1000, 2)).astype(np.float32)
    x0, y0, wx, wy = om.gather_taps(grid, W, H)
    fx = (grid[:, 0].astype(np.float64) + 1) * W / 2 - 0.5
    assert np.all(np.abs(x0 + wx - fx) < 1e-5)
    assert np.all((wx >= 0) & (wx < 1) & (wy >= 0) & (wy < 1))


# ---------------------------------------------------------------- upfirdn2x

def naive_upfirdn(x, W, C, k, up, pad0, pad1):
    """the reference's naive upfirdn2d (tests/test_ops.cpp:16-39): zero-stuff,
    pad, 4x4 correlation with double accumulation; x (C, W, W)"""
    UW = W * up
    PW = UW + pad0 + pad1
    OW = PW - 4 + 1
    pad = np.zeros((C, PW, PW), np.float64)
    pad[:, pad0:pad0 + UW:up, pad0:pad0 + UW:up] = x
    out = np.zeros((C, OW, OW), np.float64)
    for a in range(4):
        for b in range(4):
            out += k[a * 4 + b] * pad[:, a:a + OW, b:b + OW]
    return out.astype(np.float32)


def test_upfirdn2x_kat(om):
    """tests/test_ops.cpp:82-106: up=2 pad (2,1), W=6, C=3, [1,3,3,1] kernel,
    |err| < 1e-5 against the naive reference"""
    W, C = 6, 3
    x = rng(42).standard_normal((C, W, W)).astype(np.float32)
    k1 = np.array([1, 3, 3, 1], np.float64)
    kern = (np.outer(k1, k1) / 64.0).astype(np.float32).ravel()
    got = om.upfirdn2x(x, kern)
    ref = naive_upfirdn(x, W, C, kern, 2, 2, 1)
    assert got.shape == ref.shape == (C, 12, 12)
    assert np.abs(got - ref).max() < 1e-5
    # the decoder's x4 kernel against torch's upfirdn2d formulation
    k4 = kern * 4
    tv = torch_upfirdn2d(torch.tensor(x[None], dtype=torch.float64),
                         torch.tensor(k4.reshape(4, 4), dtype=torch.float64), up=2, pad=(2, 1))
    assert np.abs(om.upfirdn2x(x, k4) - tv[0].numpy()).max() < 1e-5


def test_upfirdn2x_nonsquare_batch(om):
    """GGML_OP_UPFIRDN2X correlates with k4[i + 4j] (i along x); upfirdn2d
    convolves, so an asymmetric kernel is passed flipped to the torch form
    (the decoder's kernels are symmetric, where both agree)"""
    x = rng(3).standard_normal((2, 3, 5, 7)).astype(np.float32)
    k = rng(4).standard_normal(16).astype(np.float32)
    got = om.upfirdn2x(x, k)
    kt = torch.flip(torch.tensor(k.reshape(4, 4), dtype=torch.float64), [0, 1])
    tv = torch_upfirdn2d(torch.tensor(x.reshape(1, 6, 5, 7), dtype=torch.float64), kt, up=2, pad=(2, 1))
    assert np.abs(got.reshape(6, 10, 14) - tv[0].numpy()).max() < 1e-5


# ---------------------------------------------------------------- pointwise

def test_subpix_cl_is_pixel_shuffle(om):
    g = rng(5)
    nb, W, H, OC = 2, 3, 4, 8
    y4 = g.standard_normal((nb, W * H, 4 * OC)).astype(np.float32)
    b = g.standard_normal(OC).astype(np.float32)
    got = om.subpix_lrelu_cl(y4, b, W, H)
    # numpy pixel shuffle: (nb, H, W, by, bx, OC) -> (nb, 2H, 2W, OC)
    t = y4.reshape(nb, H, W, 2, 2, OC).astype(np.float64) + b
    t = t.transpose(0, 1, 3, 2, 4, 5).reshape(nb, 2 * H * 2 * W, OC)
    want = np.where(t > 0, t, 0.2 * t)
    assert np.abs(got - want).max() < 1e-6


def test_subpix_sp_is_pixel_shuffle(om):
    g = rng(6)
    W, H, OC = 5, 3, 4
    g0 = g.standard_normal((2 * OC, H, W)).astype(np.float32)
    g1 = g.standard_normal((2 * OC, H, W)).astype(np.float32)
    b = g.standard_normal(OC).astype(np.float32)
    got = om.subpix_lrelu(g0, g1, b)
    cls = np.stack([g0[:OC], g0[OC:], g1[:OC], g1[OC:]]).reshape(2, 2, OC, H, W)  # by, bx
    t = cls.transpose(2, 3, 0, 4, 1).reshape(OC, 2 * H, 2 * W).astype(np.float64) + b[:, None, None]
    want = np.where(t > 0, t, 0.2 * t)
    assert np.abs(got - want).max() < 1e-6


def test_bias_lrelu_clsp_flowgrid(om):
    g = rng(8)
    x = g.standard_normal((2, 6, 5, 4)).astype(np.float32)
    b = g.standard_normal(6).astype(np.float32)
    want = x + b[None, :, None, None]
    want = np.where(want > 0, want, np.float32(0.2) * want)
    assert np.array_equal(om.bias_lrelu(x, b, 2), want.astype(np.float32))
    xc = g.standard_normal((7, 6)).astype(np.float32)
    wc = xc + b
    assert np.array_equal(om.bias_lrelu(xc, b, 0), np.where(wc > 0, wc, np.float32(0.2) * wc))
    cl = g.standard_normal((11, 6)).astype(np.float32)
    m = g.random(11).astype(np.float32)
    o = g.standard_normal((6, 11)).astype(np.float32)
    assert np.array_equal(om.clsp(cl, m), (cl * m[:, None]).T)
    want = (cl * m[:, None]).T + o * (np.float32(1) - m)[None]
    assert np.array_equal(om.clsp(cl, m, o), want.astype(np.float32))
    fl = g.standard_normal((3, 4, 5)).astype(np.float32) * 3
    xs = g.standard_normal((2, 20)).astype(np.float32)
    got = om.flow_grid(fl, xs)
    f = fl.reshape(3, 20).astype(np.float64)
    assert np.abs(got[0] - (np.tanh(f[0]) + xs[0])).max() < 1e-6
    assert np.abs(got[1] - (np.tanh(f[1]) + xs[1])).max() < 1e-6
    assert np.abs(got[2] - 1 / (1 + np.exp(-f[2]))).max() < 1e-6


# ---------------------------------------------------------------- conv pieces

def test_conv2d_direct_and_im2col_vs_torch(om):
    g = rng(9)
    x = g.standard_normal((6, 7, 5)).astype(np.float32)
    w = g.standard_normal((4, 6, 3, 3)).astype(np.float32)
    want = F.conv2d(torch.tensor(x[None], dtype=torch.float64), torch.tensor(w, dtype=torch.float64),
                    padding=1)[0].numpy()
    assert np.abs(om.conv2d_direct(x, w, 1) - want).max() < 1e-5
    # cf im2col + GEMM with the acf matrix computes the same conv
    x_cl = np.ascontiguousarray(x.transpose(1, 2, 0).reshape(1, 35, 6))
    im = om.im2col_cf(x_cl, 5, 7)
    ac = np.empty((4, 54), np.float32)
    W = np.ascontiguousarray(w)
    om.lib().orc_acf(om._p(W), 4, 6, om._p(ac))
    y = (im[0].astype(np.float64) @ ac.T.astype(np.float64)).T.reshape(4, 7, 5)
    assert np.abs(y - want).max() < 1e-5
    # im2col_cf rows r = ic + IC*(kw + 3kh) against torch unfold (rows ic*9 + kh*3 + kw)
    un = F.unfold(torch.tensor(x[None]), 3, padding=1)[0].numpy()   # (54, 35)
    un = un.reshape(6, 3, 3, 35).transpose(1, 2, 0, 3).reshape(54, 35)  # (kh, kw, ic)
    assert np.array_equal(im[0].T, un)


def test_saug_closed_form(om):
    g = rng(10)
    OC, IC = 5, 7
    W = g.standard_normal((OC, IC, 3, 3)).astype(np.float32)
    sa = np.empty((OC, IC + 1), np.float32)
    om.lib().orc_saug(om._p(W), OC, IC, 9, om._p(sa))
    want = 0.5 * (W.astype(np.float64) ** 2).sum((2, 3))
    assert np.array_equal(sa[:, :IC], want.astype(np.float32))
    assert np.all(sa[:, IC] == np.float32(0.5e-8))
    # den = sqrt(S.[s^2;1]) equals the StyleGAN2 demod norm / sqrt(2)
    s = g.standard_normal(IC)
    den = np.sqrt(sa[:, :IC].astype(np.float64) @ (s * s) + sa[:, IC])
    w = W.astype(np.float64) * s[None, :, None, None]
    ref = np.sqrt((w * w).sum((1, 2, 3)) + 1e-8) / math.sqrt(2)
    assert np.abs(den - ref).max() < 1e-6 * ref.max()


@pytest.mark.parametrize("IC,OC,H,W", [(4, 4, 5, 5), (3, 6, 4, 7)])
def test_composed_subpixel_upconv(om, IC, OC, H, W):
    """conv with the composed per-parity kernels + pixel shuffle ==
    conv_transpose2d(stride 2) followed by Blur(pad (1,1)), in torch"""
    g = rng(IC * 10 + W)
    Wt = g.standard_normal((OC, IC, 3, 3)).astype(np.float32)
    k1 = np.array([1, 3, 3, 1], np.float64)
    bk = (np.outer(k1, k1) / 64 * 4).astype(np.float32)
    x = g.standard_normal((IC, H, W)).astype(np.float32)
    ts = np.empty((4 * OC, 9 * IC), np.float32)
    om.lib().orc_tsubcf(om._p(Wt), om._p(np.ascontiguousarray(bk.ravel())), OC, IC, om._p(ts))
    x_cl = np.ascontiguousarray(x.transpose(1, 2, 0).reshape(1, H * W, IC))
    y4 = (om.im2col_cf(x_cl, W, H)[0].astype(np.float64) @ ts.T.astype(np.float64))  # (HW, 4OC)
    y = y4.reshape(H, W, 2, 2, OC).transpose(4, 0, 2, 1, 3).reshape(OC, 2 * H, 2 * W)
    xt = torch.tensor(x[None], dtype=torch.float64)
    wt = torch.tensor(Wt, dtype=torch.float64)
    ref = F.conv_transpose2d(xt, wt.transpose(0, 1), stride=2)
    ref = torch_upfirdn2d(ref, torch.tensor(bk, dtype=torch.float64), pad=(1, 1))[0].numpy()
    assert ref.shape == y.shape
    assert np.abs(y - ref).max() < 1e-5 * max(1, np.abs(ref).max())
