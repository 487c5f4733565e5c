"""The real-weight path on the GPU: a decoder loaded from a motion_ae GGUF
checkpoint (tpmd_load_gguf, and tp::motion_dec over tp::gguf_weight_source)
decodes exactly what the same weights handed over by name decode, for f32
and f16 files; a wrong architecture is refused (src/gguf_load.cpp:94-100)."""
import os
import subprocess

import numpy as np
import pytest

import gguf_writer
import synth
import tpmd
from test_gpu_shim import IC, OC, SHIM, write_blob

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ftype", ["f32", "f16"])
def test_gguf_decoder_matches_named_weights(torch_cuda, tmp_path, ftype):
    raw, lat, feats = synth.workload("smooth", 3, ftype, IC, OC)
    path = tmp_path / f"motion_ae_{ftype}.gguf"
    gguf_writer.write(path, {k: (v, f16) for k, (v, f16) in raw.items()}, f16=ftype == "f16")
    a = tpmd.MotionDecoder(ftype, len(IC), IC, OC)
    a.load_gguf(path)
    b = tpmd.MotionDecoder(ftype, len(IC), IC, OC)
    b.set_weights(raw)
    for d in (a, b):
        d.prepare()
        d.build(3)
        d.set_feats(feats)
    assert np.array_equal(a.decode_batch(lat), b.decode_batch(lat))
    # the C++ shim reading the same file (tp_load's flow) agrees too
    blob, out = tmp_path / "in.blob", tmp_path / "out.f32"
    write_blob(blob, {}, feats, lat, IC, OC, ftype == "f16")
    env = dict(os.environ, TP_MDEC_BATCH="3")
    p = subprocess.run([SHIM, str(blob), str(out), "0", str(path)], env=env, capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 0, p.stderr
    got = np.fromfile(out, np.float32).reshape(4, 3, 512, 512)
    assert np.array_equal(got[:3], b.decode_batch(lat))


def test_gguf_errors(torch_cuda, tmp_path):
    raw, _, _ = synth.workload("smooth", 1, "f32", IC, OC)
    dec = tpmd.MotionDecoder("f32", len(IC), IC, OC)
    p = tmp_path / "wrong.gguf"
    gguf_writer.write(p, {k: (v, False) for k, (v, _) in raw.items()}, arch="float-fmt")
    with pytest.raises(tpmd.TpmdError, match="unexpected architecture"):
        dec.load_gguf(p)
    p = tmp_path / "partial.gguf"
    gguf_writer.write(p, {k: (v, False) for k, (v, _) in raw.items() if k != "dec.to_flows.2.bias"})
    dec.load_gguf(p)
    with pytest.raises(tpmd.TpmdError, match="missing tensor dec.to_flows.2.bias"):
        dec.prepare()
