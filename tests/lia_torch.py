"""Independent torch-CPU formulation of the LIA/StyleGAN motion decoder.

Written from the upstream model definitions (StyleGAN2 ModulatedConv2d with
demodulation, FusedLeakyReLU with its sqrt(2) gain, EqualConv2d/EqualLinear
runtime scales, Blur/Upsample via upfirdn2d, LIA's ToFlow warp and ToRGB
skip) with NONE of the reference's algebraic folds: no S_aug halving, no
sqrt(2) folded into biases or weights, no composed sub-pixel kernel, no
channel-last graph.  Agreement with the oracle therefore pins the folds.
"""
import math

import torch
import torch.nn.functional as F

SQRT2 = math.sqrt(2.0)


def upfirdn2d(x, k, up=1, pad=(0, 0)):
    """x (B, C, H, W); k (kh, kw) FIR; zero-stuff by `up`, pad, convolve."""
    B, C, H, W = x.shape
    if up > 1:
        z = x.new_zeros(B, C, H * up, W * up)
        z[:, :, ::up, ::up] = x
        x = z
    x = F.pad(x, (pad[0], pad[1], pad[0], pad[1]))
    w = torch.flip(k, [0, 1]).to(x.dtype)[None, None].repeat(C, 1, 1, 1)
    return F.conv2d(x, w, groups=C)


def fused_lrelu(x, b):
    return F.leaky_relu(x + b.view(1, -1, 1, 1), 0.2) * SQRT2


def modulated_conv(x, W, style, demod=True, up=False, blur=None):
    """x (1, IC, H, W); W raw (OC, IC, k, k); style (IC,)."""
    OC, IC, k, _ = W.shape
    w = W * (1.0 / math.sqrt(IC * k * k)) * style.view(1, IC, 1, 1)
    if demod:
        d = torch.rsqrt((w * w).sum(dim=(1, 2, 3)) + 1e-8)
        w = w * d.view(OC, 1, 1, 1)
    if up:
        y = F.conv_transpose2d(x, w.transpose(0, 1), stride=2, padding=0)
        return upfirdn2d(y, blur, pad=(1, 1))
    return F.conv2d(x, w, padding=k // 2)


def equal_linear(x, W, b):
    return F.linear(x, W * (1.0 / math.sqrt(W.shape[1])), b)


def decode(raw, latent, feats, ic, oc, n_stages=None, taps=None):
    """raw: name -> (array, _) raw synthetic weights; latent (512,); feats[j]
    (r*r, C) pixel-major.  Returns the image (3, R, R) as float64 numpy."""
    dt = torch.float64
    T = {k: torch.tensor(v[0], dtype=dt) for k, v in raw.items()}
    w = torch.tensor(latent, dtype=dt)
    ns = len(ic) if n_stages is None else n_stages

    def style(base):
        return equal_linear(w[None], T[base + ".modulation.weight"], T[base + ".modulation.bias"])[0]

    def styled(x, base, up=False):
        s = style(base + ".conv")
        W = T[base + ".conv.weight"][0]
        blur = T[base + ".conv.blur.kernel"] if up else None
        y = modulated_conv(x, W, s, demod=True, up=up, blur=blur)
        return fused_lrelu(y, T[base + ".activate.bias"].reshape(-1))

    out = T["dec.input.input"]
    out = styled(out, "dec.conv1")
    if taps is not None:
        taps["conv1_4"] = out[0].numpy()
    skip = skip_flow = None
    for j in range(ns):
        r = 8 << j
        out = styled(out, f"dec.convs.{2 * j}", up=True)
        if taps is not None:
            taps[f"r{r}.conv1"] = out[0].numpy()
        out = styled(out, f"dec.convs.{2 * j + 1}")
        if taps is not None:
            taps[f"r{r}.conv2"] = out[0].numpy()
        fb = f"dec.to_flows.{j}"
        fs = style(fb + ".conv")
        fl = modulated_conv(out, T[fb + ".conv.weight"][0], fs, demod=False)
        fl = fl + T[fb + ".bias"]
        if skip_flow is not None:
            fl = fl + upfirdn2d(skip_flow, T[fb + ".upsample.kernel"], up=2, pad=(2, 1))
        skip_flow = fl
        lin = torch.linspace(-1, 1, r, dtype=dt)
        gy, gx = torch.meshgrid(lin, lin, indexing="ij")
        flow = torch.tanh(fl[:, 0:2]).permute(0, 2, 3, 1) + torch.stack([gx, gy], -1)[None]
        mask = torch.sigmoid(fl[:, 2:3])
        feat = torch.tensor(feats[j], dtype=dt).reshape(r, r, -1).permute(2, 0, 1)[None]
        warp = F.grid_sample(feat, flow, mode="bilinear", padding_mode="zeros",
                             align_corners=False) * mask
        trunk = warp + out * (1 - mask)
        rb = f"dec.to_rgbs.{j}"
        Wr = T[rb + ".conv.0.weight"]
        rgb = F.conv2d(warp, Wr * (1.0 / math.sqrt(Wr.shape[1])))
        rgb = fused_lrelu(rgb, T[rb + ".conv.1.bias"]) + T[rb + ".bias"]
        if skip is not None:
            rgb = rgb + upfirdn2d(skip, T[rb + ".upsample.kernel"], up=2, pad=(2, 1))
        skip = rgb
        if taps is not None:
            taps[f"r{r}.flowmap"] = fl[0].numpy()
            taps[f"r{r}.warp"] = warp[0].numpy()
            taps[f"r{r}.out"] = trunk[0].numpy()
            taps[f"r{r}.rgb"] = rgb[0].numpy()
        out = trunk
    return skip[0].numpy()


def encode(raw, image, cin, cout, taps=None):
    """Upstream LIA EncoderApp + fc chain + Direction (EqualConv2d runtime
    scales, FusedLeakyReLU x sqrt2, ResBlock (conv2 + skip) / sqrt2, Blur as
    upfirdn2d with the normalised [1,3,3,1] kernel), float64, NO folds.
    raw: name -> (array, _) raw synthetic encoder weights; image (3, H, W).
    Returns (appearance, lambda, motion, pyramid list conv0..conv7) numpy."""
    dt = torch.float64
    T = {k: torch.tensor(v[0], dtype=dt) for k, v in raw.items()}

    def eqconv(x, W, stride, pad):
        fan_in = W.shape[1] * W.shape[2] * W.shape[3]
        return F.conv2d(x, W * (1.0 / math.sqrt(fan_in)), stride=stride, padding=pad)

    b0 = "enc.net_app.convs"
    x = torch.tensor(image, dtype=dt)[None]
    x = fused_lrelu(eqconv(x, T[f"{b0}.0.0.weight"], 1, 0), T[f"{b0}.0.1.bias"])
    pyr = [x]
    for i in range(1, len(cin) + 1):
        b = f"{b0}.{i}"
        out = fused_lrelu(eqconv(x, T[f"{b}.conv1.0.weight"], 1, 1), T[f"{b}.conv1.1.bias"])
        out = upfirdn2d(out, T[f"{b}.conv2.0.kernel"], pad=(2, 2))
        out = fused_lrelu(eqconv(out, T[f"{b}.conv2.1.weight"], 2, 0), T[f"{b}.conv2.2.bias"])
        skip = eqconv(upfirdn2d(x, T[f"{b}.skip.0.kernel"], pad=(1, 1)), T[f"{b}.skip.1.weight"], 2, 0)
        x = (out + skip) / SQRT2
        pyr.append(x)
    app = eqconv(x, T[f"{b0}.{len(cin) + 1}.weight"], 1, 0).reshape(-1)
    h = app
    for i in range(5):
        h = equal_linear(h[None], T[f"enc.fc.{i}.weight"], T[f"enc.fc.{i}.bias"])[0]
        if taps is not None:
            taps[f"menc.fc{i}"] = h.numpy()
    motion = T["dec.direction.Q"] @ h
    return app.numpy(), h.numpy(), motion.numpy(), [p[0].numpy() for p in pyr]
