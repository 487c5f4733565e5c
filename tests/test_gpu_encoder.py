"""Motion encoder (tpme_*) on the GPU against the CPU oracle
(oracle/menc.py, the reference's folded graph, src/motion_enc.cpp:50-184):
every pyramid level, appearance, lambda and motion; f32 rel-L2 <= 1e-4, f16
rel-L2 <= 1e-2 with cosine >= 0.9999.  Then the encoder's device feats drive
the decoder exactly as the same feats uploaded from the host do."""
import numpy as np
import pytest

import gguf_writer
import synth
import tpmd
from metrics import cosine, rel_l2

pytestmark = pytest.mark.gpu

SMALL_IN = (32, 32, 64, 64, 64, 64, 64)
SMALL_OUT = (32, 64, 64, 64, 64, 64, 64)


def _close(ftype, got, want, what):
    e = rel_l2(got, want)
    if ftype == "f32":
        assert e <= 1e-4, (what, e)
    else:
        assert e <= 1e-2 and cosine(got, want) >= 0.9999, (what, e, cosine(got, want))


def _run(oracle_menc, ftype, cin, cout):
    raw = synth.enc_raw_weights(1004, ftype, cin, cout)
    img = synth.image(1005)
    want = oracle_menc.Encoder(raw, ftype, cin, cout).run(img)
    enc = tpmd.MotionEncoder(ftype, cin, cout)
    enc.set_weights(raw)
    enc.prepare()
    got = enc.run(img)
    return enc, got, want


def _check_all(ftype, enc, got, want):
    for l in range(enc.n_blocks + 1):
        t = want["taps"][f"menc.conv{l}"]
        _close(ftype, enc.level(l), t.reshape(t.shape[0], -1).T, f"menc.conv{l}")
    for k in ("appearance", "lambda", "motion"):
        _close(ftype, got[k], want[k], k)
    for j, f in enumerate(got["feats"]):
        assert f.shape == want["feats"][j].shape
        _close(ftype, f, want["feats"][j], f"feat{j}")


@pytest.mark.parametrize("ftype", ["f32", "f16"])
def test_encoder_small(oracle_menc, torch_cuda, ftype):
    enc, got, want = _run(oracle_menc, ftype, SMALL_IN, SMALL_OUT)
    _check_all(ftype, enc, got, want)


@pytest.mark.parametrize("ftype", ["f16", "f32"])
def test_encoder_reference_widths(oracle_menc, torch_cuda, ftype):
    enc, got, want = _run(oracle_menc, ftype, synth.ENC_IN, synth.ENC_OUT)
    _check_all(ftype, enc, got, want)


def test_encoder_feeds_decoder(torch_cuda):
    """device feats from tpme_feat == the same values through tpmd_set_feats"""
    torch = torch_cuda
    raw_e = synth.enc_raw_weights(1004, "f16")
    enc = tpmd.MotionEncoder("f16")
    enc.set_weights(raw_e)
    enc.prepare()
    img = torch.from_numpy(synth.image(1005)).cuda()
    out = enc.run(img)                                   # device image
    raw_d, lat, _ = synth.workload("smooth", 3, "f16")
    decs = []
    for _ in range(2):
        d = tpmd.MotionDecoder("f16", 7)
        d.set_weights(raw_d)
        d.prepare()
        d.build(4)
        decs.append(d)
    decs[0].set_feats_device(enc.feats_device())
    decs[1].set_feats(out["feats"])
    a, b = decs[0].decode_batch(lat), decs[1].decode_batch(lat)
    assert np.isfinite(a).all() and np.array_equal(a, b)


def test_encoder_error_contract(torch_cuda):
    enc = tpmd.MotionEncoder("f32", SMALL_IN, SMALL_OUT)
    with pytest.raises(tpmd.TpmdError, match="not prepared"):
        enc.run(np.zeros((3, 512, 512), np.float32))
    with pytest.raises(tpmd.TpmdError, match="missing tensor enc.net_app.convs.0.0.weight"):
        enc.prepare()
    z = np.zeros(1, np.float32)
    assert tpmd.lib().tpme_set_weight(enc.h, b"enc.nope", z.ctypes.data, 1, 0) == -1
    assert b"unknown encoder tensor enc.nope" in tpmd.lib().tpme_last_error(enc.h)


@pytest.mark.parametrize("ftype", ["f32", "f16"])
def test_encoder_from_gguf(torch_cuda, tmp_path, ftype):
    """tpme_load_gguf on a motion_ae file holding the encoder tensors gives
    the encoder of the same named weights, bit for bit"""
    raw = synth.enc_raw_weights(1004, ftype, SMALL_IN, SMALL_OUT)
    path = tmp_path / f"motion_ae_enc_{ftype}.gguf"
    gguf_writer.write(path, {k: (v, f16) for k, (v, f16) in raw.items()}, f16=ftype == "f16")
    img = synth.image(1005)
    outs = []
    for use_file in (False, True):
        enc = tpmd.MotionEncoder(ftype, SMALL_IN, SMALL_OUT)
        if use_file:
            enc.load_gguf(path)
        else:
            enc.set_weights(raw)
        enc.prepare()
        outs.append(enc.run(img))
    for k in ("appearance", "lambda", "motion"):
        assert np.array_equal(outs[0][k], outs[1][k]), k
    for a, b in zip(outs[0]["feats"], outs[1]["feats"]):
        assert np.array_equal(a, b)
