"""Decoder-level pins of the CPU oracle:
  * exact (parity) graph vs an independent torch formulation of the upstream
    model (no folds), per stage tap;
  * fast channel-last graph vs exact graph in f32 (the parity bridge,
    rel-L2 <= 1e-4 per stage tap);
  * fast f16 vs fast f32 (frame cosine / SSIM).
End-to-end comparisons use the well-conditioned "smooth" workload: with the
i.i.d. workload the warp amplifies rounding-level flow differences by ~r/2
per stage (f32 vs f64 differ by rel-L2 ~0.35 at 512x512), so there the
stage-level test below feeds both sides identical stage inputs."""
import numpy as np
import pytest

import lia_torch
import synth
from metrics import cosine, rel_l2, ssim, to_sp

SMALL_IC = (64, 64, 64, 64, 32, 32, 32)
SMALL_OC = (64, 64, 64, 32, 32, 32, 32)


@pytest.fixture(scope="module")
def small(om):
    raw, lat, feats = synth.workload("smooth", 3, "f32", SMALL_IC, SMALL_OC)
    dec = om.Decoder(raw, "f32", SMALL_IC, SMALL_OC)
    dec.set_feats(feats)
    return raw, feats, lat, dec


def test_exact_graph_vs_torch_model(small):
    raw, feats, lat, dec = small
    img, taps = dec.decode_exact(lat[0])
    ttaps = {}
    want = lia_torch.decode(raw, lat[0], feats, SMALL_IC, SMALL_OC, taps=ttaps)
    assert img.shape == want.shape == (3, 512, 512)
    for k, v in ttaps.items():
        assert rel_l2(taps[k], v) < 1e-4, k
    assert rel_l2(img, want) < 1e-4


def test_fast_graph_vs_exact_graph_f32(small):
    raw, feats, lat, dec = small
    imgs, ft = dec.decode_fast(lat, want_taps=True)
    for b in range(lat.shape[0]):
        img, et = dec.decode_exact(lat[b])
        for k, v in et.items():
            if k == "r8.grid" or k.endswith(".grid") or k == "conv1_4":
                continue
            r = int(k.split(".")[0][1:])
            got = to_sp(ft[k], r)[b]
            assert rel_l2(got, v) < 1e-4, (b, k, rel_l2(got, v))
        assert rel_l2(imgs[b], img) < 1e-4


def test_fast_graph_f16_close_to_f32(om):
    raw16, lat, feats = synth.workload("smooth", 2, "f16", SMALL_IC, SMALL_OC)
    d16 = om.Decoder(raw16, "f16", SMALL_IC, SMALL_OC)
    d32 = om.Decoder(raw16, "f32", SMALL_IC, SMALL_OC)
    d16.set_feats(feats)
    d32.set_feats(feats)
    a = d16.decode_fast(lat)
    b = d32.decode_fast(lat)
    for i in range(2):
        assert cosine(a[i], b[i]) > 0.999
        assert ssim(a[i], b[i]) > 0.99


def test_reference_channels_truncated(om):
    """the reference channel widths (512 at r8..r32), 3 stages, vs torch"""
    ic, oc = synth.REF_IC[:3], synth.REF_OC[:3]
    raw, lat, feats = synth.workload("iid", 1, "f32", ic, oc)
    dec = om.Decoder(raw, "f32", ic, oc)
    dec.set_feats(feats)
    img, _ = dec.decode_exact(lat[0])
    want = lia_torch.decode(raw, lat[0], feats, ic, oc)
    assert rel_l2(img, want) < 1e-4
    fast = dec.decode_fast(lat)
    assert rel_l2(fast[0], img) < 1e-4


def test_iid_workload_stage_by_stage(om):
    """i.i.d. workload: each fast-graph stage fed the EXACT graph's stage
    input agrees with the exact stage output (rel-L2 <= 1e-4 per tap)"""
    raw, lat, feats = synth.workload("iid", 1, "f32", SMALL_IC, SMALL_OC)
    dec = om.Decoder(raw, "f32", SMALL_IC, SMALL_OC)
    dec.set_feats(feats)
    _, et = dec.decode_exact(lat[0], n_stages=4)
    import numpy as np
    s = lat[:1]
    x = np.ascontiguousarray(et["conv1_4"].reshape(SMALL_IC[0], 16).T[None])
    for j in range(4):
        r = 8 << j
        b1, b2 = f"dec.convs.{2 * j}", f"dec.convs.{2 * j + 1}"
        s1 = dec.style_of(b1 + ".conv", s)
        s2 = dec.style_of(b2 + ".conv", s)
        c1 = dec._styled_conv_up_cl(x, r // 2, r // 2, b1, s1, dec.demod_den(b1 + ".conv.weight", s1))
        assert rel_l2(to_sp(c1, r)[0], et[f"r{r}.conv1"]) < 1e-4
        cin = np.ascontiguousarray(et[f"r{r}.conv1"].reshape(SMALL_OC[j], -1).T[None])
        out = dec._styled_conv_cl(cin, r, r, b2, s2, dec.demod_den(b2 + ".conv.weight", s2))
        assert rel_l2(to_sp(out, r)[0], et[f"r{r}.conv2"]) < 1e-4
        x = np.ascontiguousarray(et[f"r{r}.out"].reshape(SMALL_OC[j], -1).T[None])
