"""The C++ tp::motion_dec shim (host/motion_dec.h), driven like the
reference's generation loop (src/pipeline.cpp:153-185) by host/shim_check:
its frames equal the Python binding's bit for bit (same library, same
kernels), its single-frame decode() equals decode_batch's frame, and the
tensor list it walks matches the synthetic checkpoint's names."""
import os
import struct
import subprocess

import numpy as np
import pytest

import synth
import tpmd

pytestmark = pytest.mark.gpu

IC = (64, 64, 64, 32, 32, 32, 32)
OC = (64, 64, 32, 32, 32, 32, 32)
SHIM = os.path.join(os.path.dirname(tpmd.LIB_PATH), "shim_check")


def write_blob(path, raw, feats, styles, ic, oc, f16):
    with open(path, "wb") as f:
        f.write(b"TPMDBLOB")
        f.write(struct.pack("<I", len(ic)))
        f.write(struct.pack(f"<{len(ic)}i", *ic))
        f.write(struct.pack(f"<{len(oc)}i", *oc))
        f.write(struct.pack("<II", int(f16), len(raw)))
        for name, (arr, f16_file) in raw.items():
            nb = name.encode()
            a = np.ascontiguousarray(arr, np.float32).ravel()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<BQ", int(f16_file), a.size))
            f.write(a.tobytes())
        for x in feats:
            f.write(np.ascontiguousarray(x, np.float32).tobytes())
        f.write(struct.pack("<I", styles.shape[0]))
        f.write(np.ascontiguousarray(styles, np.float32).tobytes())


@pytest.mark.parametrize("ftype", ["f16", "f32"])
def test_shim_matches_binding(torch_cuda, tmp_path, ftype):
    raw, lat, feats = synth.workload("smooth", 5, ftype, IC, OC)
    blob, out = tmp_path / "in.blob", tmp_path / "out.f32"
    write_blob(blob, raw, feats, lat, IC, OC, ftype == "f16")
    env = dict(os.environ, TP_MDEC_BATCH="2")      # 3 launches, the last one padded
    p = subprocess.run([SHIM, str(blob), str(out)], env=env, capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 0, p.stderr
    R = 512
    got = np.fromfile(out, np.float32).reshape(6, 3, R, R)
    dec = tpmd.MotionDecoder(ftype, len(IC), IC, OC)
    assert sorted(n for n, _, _ in dec.weight_names()) == sorted(raw)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(2)
    dec.set_feats(feats)
    want = np.concatenate([dec.decode_batch(lat[t:t + 2]) for t in range(0, 5, 2)])
    assert np.array_equal(got[:5], want)
    assert np.array_equal(got[5], want[0])


def test_shim_errors(torch_cuda, tmp_path):
    raw, lat, feats = synth.workload("smooth", 1, "f32", IC, OC)
    del raw["dec.to_rgbs.3.bias"]
    blob = tmp_path / "in.blob"
    write_blob(blob, raw, feats, lat, IC, OC, False)
    p = subprocess.run([SHIM, str(blob), str(tmp_path / "o")], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 1 and "missing tensor dec.to_rgbs.3.bias" in p.stderr


def test_shim_encoder_to_decoder(torch_cuda, tmp_path):
    """the generation flow through both C++ shims, weights from one motion_ae
    GGUF holding enc.* and dec.*: tp::motion_enc::run on an image, its
    menc_result into tp::motion_dec::set_feats, then decode_batch — equal,
    bit for bit, to MotionEncoder + MotionDecoder through the binding"""
    import gguf_writer
    ftype = "f16"
    raw, lat, feats = synth.workload("smooth", 3, ftype, IC, OC)
    # the encoder channel plan that produces feats with OC[j] channels
    cout = tuple(OC[5 - i] for i in range(6)) + (OC[0],)
    cin = (OC[6],) + cout[:6]
    raw_e = synth.enc_raw_weights(1004, ftype, cin, cout)
    gguf = tmp_path / "motion_ae.gguf"
    gguf_writer.write(gguf, {**raw, **raw_e}, f16=True)
    img = synth.image(1005)
    img_path = tmp_path / "image.f32"
    img.tofile(img_path)
    blob, out = tmp_path / "in.blob", tmp_path / "out.f32"
    write_blob(blob, raw, feats, lat, IC, OC, True)
    env = dict(os.environ, TP_MDEC_BATCH="2")
    p = subprocess.run([SHIM, str(blob), str(out), "0", str(gguf), str(img_path)], env=env,
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    R = 512
    got = np.fromfile(out, np.float32)
    frames = got[:4 * 3 * R * R].reshape(4, 3, R, R)
    app, lam, mot = np.split(got[4 * 3 * R * R:], [512, 532])
    enc = tpmd.MotionEncoder(ftype, cin, cout)
    enc.set_weights(raw_e)
    enc.prepare()
    r = enc.run(img)
    assert np.array_equal(app, r["appearance"]) and np.array_equal(lam, r["lambda"])
    assert np.array_equal(mot, r["motion"])
    dec = tpmd.MotionDecoder(ftype, len(IC), IC, OC)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(2)
    dec.set_feats(r["feats"])
    want = np.concatenate([dec.decode_batch(lat[t:t + 2]) for t in range(0, 3, 2)])
    assert np.array_equal(frames[:3], want)


def test_shim_serves_the_tap_plan(torch_cuda, tmp_path):
    """tools/tp-parity's flow through the shim: build(be, true), then decode
    with a tap sink (a tap_writer with add_f32 and a prefix): every tap lands
    in the writer under the sink's prefix, the same bits as the binding's
    tpmd_decode_taps"""
    raw, lat, feats = synth.workload("smooth", 2, "f16", IC, OC)
    blob, out, tdir = tmp_path / "in.blob", tmp_path / "out.f32", tmp_path / "taps"
    tdir.mkdir()
    write_blob(blob, raw, feats, lat, IC, OC, True)
    env = dict(os.environ, TP_MDEC_BATCH="2", TPMD_SHIM_TAPS=str(tdir))
    p = subprocess.run([SHIM, str(blob), str(out)], env=env, capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    got = np.fromfile(out, np.float32).reshape(-1, 3, 512, 512)
    dec = tpmd.MotionDecoder("f16", len(IC), IC, OC)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(2)
    dec.set_feats(feats)
    img, taps = dec.decode_taps(lat[0])
    assert np.array_equal(got[-1], img)
    meta = [l.split() for l in (tdir / "meta.txt").read_text().splitlines()]
    assert [m[0] for m in meta] == ["mdec.f0." + n for n in taps]
    for m in meta:
        name, shape = m[0][len("mdec.f0."):], tuple(int(d) for d in m[1:])
        assert shape == taps[name].shape, name
        assert np.array_equal(np.fromfile(tdir / (m[0] + ".f32"), np.float32).reshape(shape), taps[name]), name


def _steady_allocs(tmp_path, graphs):
    """heap allocations per single-frame decode() and per decode_batch() call
    of the shim in steady state, counted on the calling thread as the
    reference's zero-allocation check counts them (bench/tp-allocproof.cpp:
    121-150)"""
    import re
    raw, lat, feats = synth.workload("smooth", 8, "f16", IC, OC)
    blob, out = tmp_path / f"a{int(graphs)}.blob", tmp_path / f"a{int(graphs)}.f32"
    write_blob(blob, raw, feats, lat, IC, OC, True)
    env = dict(os.environ, TPMD_SHIM_ALLOCS="50", TPMD_GRAPHS="1" if graphs else "0")
    p = subprocess.run([SHIM, str(blob), str(out)], env=env, capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    d = re.search(r"allocs decode: (\d+) over (\d+) frames, max (\d+)", p.stdout)
    b = re.search(r"allocs decode_batch: (\d+) over (\d+) calls of (\d+) frames, max (\d+)", p.stdout)
    assert d and b, p.stdout
    per_frame = int(d.group(1)) / int(d.group(2))
    per_batch = int(b.group(1)) / int(b.group(2))
    return per_frame, per_batch, int(b.group(3))


def test_shim_steady_state_allocations(torch_cuda, tmp_path):
    """the launch chain replayed as a HIP graph makes fewer host allocations
    per decode than launch-by-launch enqueueing (the HIP runtime allocates a
    host command object per enqueued operation; the library itself none)"""
    g_frame, g_batch, B = _steady_allocs(tmp_path, True)
    d_frame, d_batch, _ = _steady_allocs(tmp_path, False)
    print(f"heap allocations, graphs: {g_frame:.1f} per decode(), {g_batch:.1f} per decode_batch({B}); "
          f"direct launches: {d_frame:.1f} per decode(), {d_batch:.1f} per decode_batch({B})")
    assert g_frame < d_frame and g_batch < d_batch
