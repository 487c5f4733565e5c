"""GGUF v3 reader of the library (host/gguf.cpp), no device needed: tensor
values and the f16 flag round-trip through a GGUF file written to the
format (exact widening of F16), metadata of every value type is walked, and
malformed files fail with the reference loader's messages
(src/gguf_load.cpp:51-197).  Every file is also read by gguf_check built
with AddressSanitizer and UndefinedBehaviorSanitizer
(host/Makefile.sanitize), which must report the same outcome and no error
of its own."""
import os
import subprocess

import numpy as np
import pytest

import gguf_writer
import synth
import tpmd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_MAKE = os.path.join(ROOT, "talking-portrait.cpp_amd", "host", "Makefile.sanitize")
SAN_BIN = os.path.join(ROOT, "talking-portrait.cpp_amd", "_build", "gguf_check_san")


@pytest.fixture(scope="module")
def san():
    subprocess.run(["make", "-s", "-f", SAN_MAKE], check=True)
    return SAN_BIN


def sanitized(bin_, path, *names):
    """(returncode, stdout) of the sanitized reader; a sanitizer finding
    fails the test"""
    env = dict(os.environ, ASAN_OPTIONS="exitcode=86:detect_leaks=1", UBSAN_OPTIONS="exitcode=87")
    p = subprocess.run([bin_, str(path), "-", *names], capture_output=True, text=True, env=env, timeout=60)
    assert p.returncode in (0, 1), (p.returncode, p.stderr[-2000:])
    assert "Sanitizer" not in p.stderr, p.stderr[-2000:]
    return p.returncode, p.stdout


def test_read_tensors_f32_and_f16(tmp_path, san):
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
    for p in (p32, p16):
        rc, out = sanitized(san, p)
        assert rc == 0 and out.count("\nok ") + out.startswith("ok ") == len(raw)


def test_f16_widening_is_exact(tmp_path):
    """every finite f16 bit pattern (subnormals included) widens exactly"""
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    vals = np.concatenate([h, h | 0x8000]).view(np.float16).astype(np.float32)
    p = tmp_path / "h.gguf"
    gguf_writer.write(p, {"x": (vals.reshape(2, -1), True)}, f16=True)
    got, f16 = tpmd.gguf_read_tensor(p, "x")
    assert f16 and np.array_equal(got.view(np.uint32), vals.view(np.uint32))


def test_metadata_of_every_type(tmp_path, san):
    """values of all 13 metadata types, arrays of scalars, of strings and of
    arrays, are walked; general.alignment places the data section"""
    kv = [("k.u8", 0, 7), ("k.i8", 1, -7), ("k.u16", 2, 700), ("k.i16", 3, -700), ("k.u32", 4, 70000),
          ("k.i32", 5, -70000), ("k.f32", 6, 0.5), ("k.bool", 7, True), ("k.str", 8, "text"),
          ("k.arr", 9, (4, [1, 2, 3])), ("k.sarr", 9, (8, ["a", "bc", ""])),
          ("k.aarr", 9, (9, [(6, [1.0, 2.0]), (0, [])])), ("k.u64", 10, 1 << 40), ("k.i64", 11, -(1 << 40)),
          ("k.f64", 12, 0.25)]
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    for align in (None, 64):
        p = tmp_path / f"kv{align}.gguf"
        gguf_writer.write(p, {"t": (a, False)}, extra_kv=kv, align=align)
        got, _ = tpmd.gguf_read_tensor(p, "t")
        assert np.array_equal(got, a.ravel())
        assert sanitized(san, p)[0] == 0


MALFORMED = [
    ("magic", "not a GGUF file"),
    ("version", "unsupported GGUF version"),
    ("empty", "not a GGUF file"),
    ("counts", "corrupt header"),
    ("kv_type", "unsupported KV type"),
    ("kv_truncated", "truncated KV section"),
    ("alignment", "general.alignment"),
    ("ndims", "corrupt tensor info"),
    ("truncated", "out of bounds"),
    ("overflow", "out of bounds"),
    ("huge_dim", "out of bounds"),
    ("type", "unsupported type"),
    ("duplicate", "duplicate tensor"),
    ("missing", "missing tensor"),
]


def _malformed(tmp_path, case):
    t = {"a": (np.ones((4, 8), np.float32), True), "b": (np.arange(5, dtype=np.float32), False)}
    p = tmp_path / f"bad_{case}.gguf"
    kw = {}
    if case == "version":
        kw["version"] = 2
    if case == "type":
        kw["bad_type"] = "a"
    if case == "duplicate":
        kw["duplicate"] = "b"
    if case == "overflow":
        # the element count wraps 64 bits: (2^32 + 1)(2^32 - 1) = 2^64 - 1
        kw["dims_override"] = {"a": [(1 << 32) + 1, (1 << 32) - 1]}
    if case == "huge_dim":
        kw["dims_override"] = {"a": [1 << 61]}
    if case == "ndims":
        kw["dims_override"] = {"a": [1] * 9}
    if case == "alignment":
        kw["align"] = 48
    if case == "kv_type":
        kw["extra_kv"] = [("k.bad", 9, (13, []))]
    gguf_writer.write(p, t, **kw)
    raw = p.read_bytes()
    if case == "magic":
        p.write_bytes(b"GGUX" + raw[4:])
    if case == "empty":
        p.write_bytes(b"")
    if case == "counts":
        p.write_bytes(raw[:8] + (1 << 62).to_bytes(8, "little") + raw[16:])
    if case == "kv_truncated":
        p.write_bytes(raw[:60])          # inside general.architecture's value
    if case == "truncated":
        p.write_bytes(raw[:-40])
    return p


@pytest.mark.parametrize("case,msg", MALFORMED)
def test_malformed_files(tmp_path, san, case, msg):
    p = _malformed(tmp_path, case)
    name = "zz" if case == "missing" else "a"
    with pytest.raises(tpmd.TpmdError, match=msg):
        tpmd.gguf_read_tensor(p, name)
    rc, out = sanitized(san, p, name)
    assert rc == 1 and msg in out, out
