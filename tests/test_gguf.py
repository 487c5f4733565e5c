"""GGUF v3 reader of the library (host/gguf.cpp), no device needed: tensor
values and the f16 flag round-trip through a GGUF file written to the
format (exact widening of F16), and malformed files fail with the
reference loader's messages (src/gguf_load.cpp:51-197)."""
import numpy as np
import pytest

import gguf_writer
import synth
import tpmd


def test_read_tensors_f32_and_f16(tmp_path):
    raw = synth.raw_weights(1000, "f32", (32,), (32,))
    p32, p16 = tmp_path / "m32.gguf", tmp_path / "m16.gguf"
    gguf_writer.write(p32, {k: (v, v.ndim >= 2) for k, (v, _) in raw.items()})
    gguf_writer.write(p16, {k: (v, v.ndim >= 2) for k, (v, _) in raw.items()}, f16=True)
    for name, (v, _) in raw.items():
        got, f16 = tpmd.gguf_read_tensor(p32, name)
        assert not f16 and np.array_equal(got, v.ravel())
        got, f16 = tpmd.gguf_read_tensor(p16, name)
        assert f16 == (v.ndim >= 2)
        want = v.astype(np.float16).astype(np.float32) if v.ndim >= 2 else v
        assert np.array_equal(got.view(np.uint32), want.ravel().view(np.uint32))


def test_f16_widening_is_exact(tmp_path):
    """every finite f16 bit pattern (subnormals included) widens exactly"""
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    vals = np.concatenate([h, h | 0x8000]).view(np.float16).astype(np.float32)
    p = tmp_path / "h.gguf"
    gguf_writer.write(p, {"x": (vals.reshape(2, -1), True)}, f16=True)
    got, f16 = tpmd.gguf_read_tensor(p, "x")
    assert f16 and np.array_equal(got.view(np.uint32), vals.view(np.uint32))


@pytest.mark.parametrize("case,msg", [
    ("magic", "not a GGUF file"),
    ("version", "unsupported GGUF version"),
    ("truncated", "out of bounds"),
    ("type", "unsupported type"),
    ("missing", "missing tensor"),
])
def test_malformed_files(tmp_path, case, msg):
    t = {"a": (np.ones((4, 8), np.float32), True), "b": (np.arange(5, dtype=np.float32), False)}
    p = tmp_path / "bad.gguf"
    gguf_writer.write(p, t, version=2 if case == "version" else 3, bad_type="a" if case == "type" else None)
    raw = p.read_bytes()
    if case == "magic":
        p.write_bytes(b"GGUX" + raw[4:])
    if case == "truncated":
        p.write_bytes(raw[:-40])
    with pytest.raises(tpmd.TpmdError, match=msg):
        tpmd.gguf_read_tensor(p, "zz" if case == "missing" else "a")
