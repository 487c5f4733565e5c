"""Minimal GGUF v3 writer for tests (little-endian, per the GGUF v3 layout the
reference's loader reads, src/gguf_load.cpp:51-197): KV strings / u32, tensor
dims in ggml order (reversed torch shape), F32 or F16 data, 32-byte aligned."""
import struct

import numpy as np

ALIGN = 32


def _s(b, text):
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def write(path, tensors, arch="float-motion-ae", f16=False, extra_kv=None, version=3,
          bad_type=None):
    """tensors: {name: (array in torch shape, store_f16)}; f16=True stores every
    tensor flagged store_f16 as F16.  bad_type: a tensor name written with
    type 8 (unsupported)."""
    kv = [("general.architecture", 8, arch)] if arch is not None else []
    kv += list(extra_kv or [])
    head = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for key, vt, val in kv:
        _s(head, key)
        head += struct.pack("<I", vt)
        if vt == 8:
            _s(head, val)
        elif vt == 4:
            head += struct.pack("<I", val)
        elif vt == 6:
            head += struct.pack("<f", val)
        else:
            raise ValueError(vt)
    blobs, off = [], 0
    for name, (arr, store16) in tensors.items():
        a = np.ascontiguousarray(arr, np.float32)
        use16 = f16 and store16
        data = (a.astype(np.float16) if use16 else a).tobytes()
        _s(head, name)
        dims = list(reversed(a.shape)) or [1]
        head += struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        gtype = 8 if name == bad_type else (1 if use16 else 0)
        head += struct.pack("<IQ", gtype, off)
        blobs.append(data)
        off += len(data)
        off = (off + ALIGN - 1) // ALIGN * ALIGN
    pad = (-len(head)) % ALIGN
    out = bytes(head) + b"\0" * pad
    for d in blobs:
        out += d + b"\0" * ((-len(d)) % ALIGN)
    with open(path, "wb") as f:
        f.write(out)
