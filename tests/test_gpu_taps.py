"""The reference's tap plan served by the GPU decoder (tpmd_decode_taps; the
shim's decode with a tap sink): one frame through the per-stage f32 kernels,
every tap in the reference's names and torch shapes (src/motion_dec.cpp:
805-883), checked tap by tap against the oracle's exact (parity) graph, which
is f32, on the well-conditioned workload: f32 rel-L2 <= 1e-4 per tap; f16
cosine >= 0.995 per tap (the f16 conv operands move the flow by ~1e-3, which
the r512 warp turns into ~0.2 % of the sampled features) and the frame at the
f16 bar, SSIM >= 0.99 and cosine >= 0.999."""
import numpy as np
import pytest

import synth
import tpmd
from metrics import cosine, rel_l2, ssim

pytestmark = pytest.mark.gpu

IC = (64, 64, 64, 64, 32, 32, 32)
OC = (64, 64, 64, 32, 32, 32, 32)


def tap_names(ns):
    names = ["conv1_4"]
    for j in range(ns):
        r = 8 << j
        names += [f"r{r}.{k}" for k in ("conv1", "conv2", "flowmap", "grid", "warp", "out", "rgb")]
    return names


@pytest.mark.parametrize("ftype", ["f32", "f16"])
def test_tap_plan_matches_exact_graph(om, torch_cuda, ftype):
    raw, lat, feats = synth.workload("smooth", 2, ftype, IC, OC)
    dec = tpmd.MotionDecoder(ftype, len(IC), IC, OC)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(2)
    dec.set_feats(feats)
    img, taps = dec.decode_taps(lat[0])
    assert list(taps) == tap_names(len(IC))
    # the oracle's exact graph is f32: the f16 decoder is compared with it too
    ref = om.Decoder(synth.workload("smooth", 2, "f32", IC, OC)[0], "f32", IC, OC)
    ref.set_feats(feats)
    want_img, want = ref.decode_exact(lat[0])
    for name, got in taps.items():
        w = want[name]
        assert got.shape == (1,) + w.shape, (name, got.shape, w.shape)
        if ftype == "f32":
            assert rel_l2(got, w) <= 1e-4, (name, rel_l2(got, w))
        else:
            assert cosine(got, w) >= 0.995, (name, cosine(got, w))
    if ftype == "f16":
        assert cosine(img, want_img) >= 0.999 and ssim(img, want_img) >= 0.99
    assert np.array_equal(img, taps[f"r{8 << (len(IC) - 1)}.rgb"][0])
    # the tap plan's frame agrees with the batched decode's
    fast = dec.decode_batch(lat[:1])[0]
    if ftype == "f32":
        assert rel_l2(img, fast) <= 1e-4
    else:
        assert cosine(img, fast) >= 0.9999
    dec.close()


def test_tap_plan_errors(torch_cuda):
    dec = tpmd.MotionDecoder("f32", 2, (64, 64), (64, 64))
    dec.set_weights(synth.raw_weights(1000, "f32", (64, 64), (64, 64)))
    dec.prepare()
    with pytest.raises(tpmd.TpmdError, match="decoder not built"):
        dec.decode_taps(np.zeros(512, np.float32))
    dec.build(1)
    with pytest.raises(tpmd.TpmdError, match="feats not set"):
        dec.decode_taps(np.zeros(512, np.float32))
    dec.close()
