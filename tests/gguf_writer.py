"""Minimal GGUF v3 writer for tests (little-endian, the GGUF v3 layout: header,
metadata key/value pairs of any of the 13 value types, tensor records with
dims in ggml order (reversed torch shape), F32 or F16 data aligned to 32
bytes or general.alignment)."""
import struct

import numpy as np

ALIGN = 32
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def _s(b, text):
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def _value(b, vt, val):
    if vt == 8:
        _s(b, val)
    elif vt == 9:                       # (element type, [values])
        et, items = val
        b += struct.pack("<IQ", et, len(items))
        for it in items:
            _value(b, et, it)
    else:
        b += struct.pack(_FMT[vt], val)


def write(path, tensors, arch="float-motion-ae", f16=False, extra_kv=None, version=3,
          bad_type=None, dims_override=None, duplicate=None, align=None):
    """tensors: {name: (array in torch shape, store_f16)}; f16=True stores every
    tensor flagged store_f16 as F16.  extra_kv: [(key, value type, value)].
    bad_type: a tensor name written with type 8 (unsupported).
    dims_override: {name: dims} written instead of the array's (the data stays
    the array's).  duplicate: a tensor name whose record is written twice.
    align: a general.alignment to write and lay the data out with."""
    kv = [("general.architecture", 8, arch)] if arch is not None else []
    if align is not None:
        kv.append(("general.alignment", 4, align))
    kv += list(extra_kv or [])
    al = align or ALIGN
    recs = list(tensors.items())
    if duplicate is not None:
        recs.append((duplicate, tensors[duplicate]))
    head = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(recs), len(kv)))
    for key, vt, val in kv:
        _s(head, key)
        head += struct.pack("<I", vt)
        _value(head, vt, val)
    blobs, off, offs = [], 0, {}
    for name, (arr, store16) in tensors.items():
        a = np.ascontiguousarray(arr, np.float32)
        data = (a.astype(np.float16) if f16 and store16 else a).tobytes()
        offs[name] = off
        blobs.append(data)
        off += len(data)
        off = (off + al - 1) // al * al
    for name, (arr, store16) in recs:
        _s(head, name)
        dims = (dims_override or {}).get(name) or list(reversed(np.shape(arr))) or [1]
        head += struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        gtype = 8 if name == bad_type else (1 if f16 and store16 else 0)
        head += struct.pack("<IQ", gtype, offs[name])
    pad = (-len(head)) % al
    out = bytes(head) + b"\0" * pad
    for d in blobs:
        out += d + b"\0" * ((-len(d)) % al)
    with open(path, "wb") as f:
        f.write(out)
