"""The HIP library against the committed golden fixtures (tests/golden/):
gather taps and values bit for bit, upfirdn2x bit for bit, and the 3-stage
decoder's frames (f32 rel-L2 <= 1e-4 against the fast and the exact graph;
f16 SSIM >= 0.99 and cosine >= 0.999)."""
import os
import sys

import numpy as np
import pytest

import tpmd
from metrics import cosine, rel_l2, ssim

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden as mg  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_gather_golden(torch_cuda):
    torch = torch_cuda
    z = np.load(os.path.join(GOLD, "gather.npz"))
    W, H = int(z["W"]), int(z["H"])
    got = tpmd.gather_taps(_dev(torch, z["grid"]), W, H)
    for a, b in zip(got, (z["x0"], z["y0"], z["wx"], z["wy"])):
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32))
    out = tpmd.gather(_dev(torch, z["feat"]), W, H, _dev(torch, z["grid"])).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), z["out"].view(np.uint32))
    f16 = _dev(torch, z["feat"].astype(np.float16))
    out = tpmd.gather(f16, W, H, _dev(torch, z["grid"])).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), z["out_f16"].view(np.uint32))


def test_upfirdn_golden(torch_cuda):
    torch = torch_cuda
    z = np.load(os.path.join(GOLD, "upfirdn.npz"))
    for x, y in (("x1", "y1"), ("x2", "y2")):
        got = tpmd.upfirdn2x(_dev(torch, z[x]), _dev(torch, z["k4"])).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), z[y].view(np.uint32))


@pytest.mark.parametrize("ftype", ["f32", "f16"])
def test_decoder_golden(torch_cuda, ftype):
    raw, lat, feats, want = mg.load_decoder_fixture()
    dec = tpmd.MotionDecoder(ftype, len(mg.IC3), mg.IC3, mg.OC3)
    dec.set_weights(raw if ftype == "f32" else mg.f16_checkpoint(raw))
    dec.prepare()
    dec.build(2)
    dec.set_feats(feats)
    got = dec.decode_batch(lat)
    if ftype == "f32":
        assert rel_l2(got, want["fast_f32"]) <= 1e-4
        assert rel_l2(got[0], want["exact_f32"]) <= 1e-4
    else:
        for b in range(2):
            assert cosine(got[b], want["fast_f16"][b]) >= 0.999
            assert ssim(got[b], want["fast_f16"][b]) >= 0.99
