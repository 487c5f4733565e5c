"""The CPU oracle reproduces the committed golden fixtures (tests/golden/,
written by tests/golden/make_golden.py): bit for bit for the gather's taps
and values and for upfirdn2x, within 1e-6 rel-L2 for the decoder frames
(BLAS blocking may differ between hosts)."""
import os
import sys

import numpy as np

from metrics import rel_l2

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden as mg  # noqa: E402

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_gather_fixture(om):
    z = np.load(os.path.join(GOLD, "gather.npz"))
    W, H, feat, grid = mg.gather_inputs()
    assert np.array_equal(feat, z["feat"]) and np.array_equal(grid, z["grid"])
    for a, b in zip(om.gather_taps(grid, W, H), (z["x0"], z["y0"], z["wx"], z["wy"])):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(om.bilinear_gather(feat, grid, W, H).view(np.uint32), z["out"].view(np.uint32))
    f16 = feat.astype(np.float16).astype(np.float32)
    assert np.array_equal(om.bilinear_gather(f16, grid, W, H).view(np.uint32), z["out_f16"].view(np.uint32))
    # some points sample outside the map (zeros padding is exercised)
    assert (z["x0"] < 0).any() and (z["x0"] >= W - 1).any()


def test_upfirdn_fixture(om):
    z = np.load(os.path.join(GOLD, "upfirdn.npz"))
    x1, x2 = mg.upfirdn_inputs()
    assert np.array_equal(om.upfirdn2x(x1, z["k4"]), z["y1"])
    assert np.array_equal(om.upfirdn2x(x2, z["k4"]), z["y2"])


def test_decoder_fixture(om):
    raw, lat, feats, want = mg.load_decoder_fixture()
    d32 = om.Decoder(raw, "f32", mg.IC3, mg.OC3)
    d32.set_feats(feats)
    assert rel_l2(d32.decode_fast(lat), want["fast_f32"]) < 1e-6
    exact, _ = d32.decode_exact(lat[0])
    assert rel_l2(exact, want["exact_f32"]) < 1e-6
    # fast and exact graphs agree (the fixture carries both)
    assert rel_l2(want["fast_f32"][0], want["exact_f32"]) < 1e-4
    d16 = om.Decoder(mg.f16_checkpoint(raw), "f16", mg.IC3, mg.OC3)
    d16.set_feats(feats)
    assert rel_l2(d16.decode_fast(lat), want["fast_f16"]) < 1e-6
