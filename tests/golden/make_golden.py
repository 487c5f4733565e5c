"""Writes the golden fixtures of this directory from the CPU oracle (itself
pinned by tests/test_oracle_*.py against torch-CPU, numpy float16, the
reference's upfirdn2d known-answer check and closed forms).

    python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  gather.npz   GGML_OP_BILINEAR_GATHER on a 16x12 map, C = 32, f32 and
               f16-valued features, 600 points ~ U(-1.3, 1.3) with jitter
               (some out of range): tap indices, tap weights, outputs
  upfirdn.npz  upfirdn2d(up=2, pad (2,1)) with the decoder's x4 kernel, the
               reference KAT's shape (W = 6, C = 3) and a batched 4x3x9x5
  decoder.npz  a 3-stage decoder (channels 32, 32x32 output, smooth
               workload, 2 frames): raw weights, latents, feats, and the
               fast-graph frames in f32 and f16 plus the exact-graph frame
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "talking-portrait.cpp_amd")]

IC3 = (32, 32, 32)
OC3 = (32, 32, 32)


def gather_inputs():
    g = np.random.default_rng(2024)
    W, H, C = 16, 12, 32
    feat = g.standard_normal((W * H, C)).astype(np.float32)
    grid = g.uniform(-1.3, 1.3, (600, 2)).astype(np.float32)
    grid += (g.uniform(-0.5, 0.5, (600, 2)) / W).astype(np.float32)
    return W, H, feat, grid


def upfirdn_inputs():
    g = np.random.default_rng(42)
    x1 = g.standard_normal((3, 6, 6)).astype(np.float32)
    x2 = g.standard_normal((4, 3, 9, 5)).astype(np.float32)
    return x1, x2


def f16_checkpoint(raw):
    """the f16 GGUF of a raw f32 checkpoint: tensors with >= 2 dims hold f16
    values (IEEE round to nearest even) and carry the f16 flag"""
    return {k: ((v.astype(np.float16).astype(np.float32), True) if v.ndim >= 2 else (v, False))
            for k, (v, _) in raw.items()}


def load_decoder_fixture():
    """(raw weights, latents, feats, expected frames) of decoder.npz"""
    z = np.load(os.path.join(HERE, "decoder.npz"))
    raw = {k[2:]: (z[k], False) for k in z.files if k.startswith("w:")}
    feats = [z[f"feat{j}"] for j in range(len(IC3))]
    return raw, z["latents"], feats, {k: z[k] for k in ("fast_f32", "fast_f16", "exact_f32")}


def main():
    from oracle import mdec as om
    import synth
    W, H, feat, grid = gather_inputs()
    f16 = feat.astype(np.float16).astype(np.float32)
    x0, y0, wx, wy = om.gather_taps(grid, W, H)
    np.savez(os.path.join(HERE, "gather.npz"), W=W, H=H, feat=feat, grid=grid, x0=x0, y0=y0, wx=wx,
             wy=wy, out=om.bilinear_gather(feat, grid, W, H), out_f16=om.bilinear_gather(f16, grid, W, H))
    x1, x2 = upfirdn_inputs()
    k4 = synth.blur_kernel().ravel()
    np.savez(os.path.join(HERE, "upfirdn.npz"), k4=k4, x1=x1, y1=om.upfirdn2x(x1, k4), x2=x2,
             y2=om.upfirdn2x(x2, k4))
    raw, lat, feats = synth.workload("smooth", 2, "f32", IC3, OC3)
    d32 = om.Decoder(raw, "f32", IC3, OC3)
    d32.set_feats(feats)
    d16 = om.Decoder(f16_checkpoint(raw), "f16", IC3, OC3)
    d16.set_feats(feats)
    arrays = {f"w:{k}": v for k, (v, _) in raw.items()}
    arrays.update({f"feat{j}": f for j, f in enumerate(feats)})
    exact, _ = d32.decode_exact(lat[0])
    np.savez_compressed(os.path.join(HERE, "decoder.npz"), latents=lat, fast_f32=d32.decode_fast(lat),
                        fast_f16=d16.decode_fast(lat), exact_f32=exact, **arrays)
    for f in ("gather.npz", "upfirdn.npz", "decoder.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
