"""The encoder oracle (oracle/menc.py, the reference's folded graph) against
the upstream torch formulation (tests/lia_torch.py: EqualConv2d scales,
FusedLeakyReLU gain, ResBlock 1/sqrt2, Blur via upfirdn2d, no folds), and the
oracle's blur against torch's upfirdn2d.  Agreement pins motion_ae_scale's
encoder folds and the graph wiring (src/motion_enc.cpp:14-160)."""
import numpy as np
import pytest

import synth
from metrics import rel_l2

torch = pytest.importorskip("torch")
import lia_torch  # noqa: E402

SMALL_IN = (8, 16, 16, 32, 32, 32, 32)
SMALL_OUT = (16, 16, 32, 32, 32, 32, 32)


def test_blur_matches_upfirdn(oracle_menc):
    g = np.random.default_rng(5)
    x = g.standard_normal((3, 11, 9)).astype(np.float32)
    k = (synth.blur_kernel() / 4).astype(np.float32)
    for pad in (1, 2):
        want = lia_torch.upfirdn2d(torch.tensor(x, dtype=torch.float64)[None],
                                   torch.tensor(k, dtype=torch.float64), pad=(pad, pad))[0].numpy()
        got = oracle_menc.blur(x, k, pad)
        assert got.shape == want.shape
        assert rel_l2(got, want) <= 1e-6


@pytest.mark.parametrize("cin,cout", [(SMALL_IN, SMALL_OUT)])
def test_encoder_matches_upstream(oracle_menc, cin, cout):
    raw = synth.enc_raw_weights(1004, "f32", cin, cout)
    img = synth.image(1005)
    got = oracle_menc.Encoder(raw, "f32", cin, cout).run(img)
    app, lam, motion, pyr = lia_torch.encode(raw, img, cin, cout)
    assert rel_l2(got["appearance"], app) <= 1e-5
    assert rel_l2(got["lambda"], lam) <= 1e-5
    assert rel_l2(got["motion"], motion) <= 1e-5
    for i, p in enumerate(pyr):
        assert rel_l2(got["taps"][f"menc.conv{i}"], p) <= 1e-5, i
    # feats[j] = conv{6-j}, pixel-major
    for j in range(len(cin)):
        p = pyr[len(cin) - 1 - j]
        assert np.array_equal(got["feats"][j], got["taps"][f"menc.conv{len(cin) - 1 - j}"].reshape(p.shape[0], -1).T)
        assert got["feats"][j].shape == ((8 << j) ** 2, p.shape[0])


def test_encoder_f16_rounding_points(oracle_menc):
    """f16 mode differs from f32 by the f16 storage of the big tensors and
    their operands only: close, and exactly equal where nothing is f16"""
    raw32 = synth.enc_raw_weights(1004, "f32", SMALL_IN, SMALL_OUT)
    raw16 = synth.enc_raw_weights(1004, "f16", SMALL_IN, SMALL_OUT)
    img = synth.image(1005)
    a = oracle_menc.Encoder(raw32, "f32", SMALL_IN, SMALL_OUT).run(img)
    b = oracle_menc.Encoder(raw16, "f16", SMALL_IN, SMALL_OUT).run(img)
    assert 0 < rel_l2(b["motion"], a["motion"]) <= 2e-2
    e16 = oracle_menc.Encoder(raw16, "f16", SMALL_IN, SMALL_OUT)
    assert not e16.isf16["enc.net_app.convs.0.0.weight"]      # 96 elements: f32
    assert e16.isf16["enc.net_app.convs.1.conv1.0.weight"] == (SMALL_IN[0] ** 2 * 9 >= 4096)
    assert e16.isf16["enc.fc.0.weight"]
