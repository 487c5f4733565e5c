"""Python binding of libtpmd.so (ctypes), the MI355X motion decoder.

A thin host mirror of the reference's tp::motion_dec interface
(src/motion_dec.h:34-47) over the C ABI of include/tpmd.h:

    dec = MotionDecoder(ftype="f16")          # tpmd_create
    dec.set_weights(raw)                       # weights_t::load, dec.* tensors
    dec.prepare()                              # motion_dec::prepare
    dec.build(batch=16)                        # motion_dec::build
    dec.set_feats(feats)                       # motion_dec::set_feats
    imgs = dec.decode_batch(styles)            # motion_dec::decode_batch

Errors raise TpmdError carrying tpmd_last_error(), the reference's
`false + err` contract.  Device buffers are torch tensors (PyTorch is used
only for device memory and streams).  The library is required: importing
this module without libtpmd.so built raises, there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtpmd.so")
HEADER = os.path.join(os.path.dirname(_HERE), "include", "tpmd.h")

W_F16_FILE = 1
W_FOLDED = 2
TAP_TRUNK, TAP_C1, TAP_OUT, TAP_FLOW, TAP_RGB = range(5)
FRAME_F32 = 0
FRAME_RGB24 = 1
FRAME_CB = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p)
TAP_CB = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int,
                          ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p)


class TpmdError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TpmdError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        P, I, I64, C = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_char_p
        sig = {
            "tpmd_abi_version": (I, []),
            "tpmd_create": (P, [I, C, I, P, P]),
            "tpmd_destroy": (None, [P]),
            "tpmd_last_error": (C, [P]),
            "tpmd_set_weight": (I, [P, C, P, I64, I]),
            "tpmd_weight_name": (C, [P, I, P, P]),
            "tpmd_load_gguf": (I, [P, C, P, ctypes.c_size_t]),
            "tpmd_gguf_read_tensor": (I64, [C, C, P, I64, P, P, ctypes.c_size_t]),
            "tpmd_prepare": (I, [P]),
            "tpmd_build": (I, [P, I]),
            "tpmd_batch": (I, [P]),
            "tpmd_out_res": (I, [P]),
            "tpmd_set_feats": (I, [P, P]),
            "tpmd_set_feats_device": (I, [P, P]),
            "tpmd_decode_batch": (I, [P, P, I, P, I]),
            "tpmd_decode": (I, [P, P, P]),
            "tpmd_decode_frames": (I64, [P, P, I64, I, P, P, P]),
            "tpmd_frames_to_rgb24": (I, [P, I, I, P, P]),
            "tpmd_sync": (I, [P]),
            "tpmd_set_stream": (I, [P, P]),
            "tpmd_set_graphs": (I, [P, I]),
            "tpmd_profile_stages": (I, [P, I]),
            "tpmd_stage_times": (I, [P, P, I]),
            "tpmd_probe_mfma_f16": (I, [I, I, P, P]),
            "tpmd_set_tap": (I, [P, I, I, P, I64]),
            "tpmd_decode_taps": (I, [P, P, P, P, P]),
            "tpmd_tap_frame_bytes": (I64, [P, I, I]),
            "tpmd_modconv": (I, [P, I, P, I, I, I, P, P, P]),
            "tpmd_modconv_static": (I, [P, I, P, I, I, I, P, P, P]),
            "tpmd_stage_tail": (I, [P, I, P, I, P, P, P, P, P, P, P, P]),
            "tpmd_stage_conv_tail": (I, [P, I, P, I, P, P, P, P, P, P, P, P, P]),
            "tpmd_gather": (I, [P, I, I, I, I, P, I64, I, I, P, P]),
            "tpmd_gather_taps": (I, [P, I, I, I64, I, P, P, P, P, P]),
            "tpmd_upfirdn2x": (I, [P, P, P, I, I, I64, P]),
            "tpmd_flow_grid": (I, [P, P, P, I64, P]),
            "tpme_create": (P, [I, C, I, P, P]),
            "tpme_destroy": (None, [P]),
            "tpme_last_error": (C, [P]),
            "tpme_weight_name": (C, [P, I, P, P]),
            "tpme_set_weight": (I, [P, C, P, I64, I]),
            "tpme_prepare": (I, [P]),
            "tpme_run": (I, [P, P, I]),
            "tpme_result": (I, [P, P, P, P]),
            "tpme_feat": (P, [P, I, P, P]),
            "tpme_level": (I64, [P, I, P]),
            "tpme_load_gguf": (I, [P, C, P, ctypes.c_size_t]),
            "tpfm_default_config": (None, [P]),
            "tpfm_read_config": (I, [C, P, P, ctypes.c_size_t]),
            "tpfm_create": (P, [I, C, P]),
            "tpfm_destroy": (None, [P]),
            "tpfm_last_error": (C, [P]),
            "tpfm_weight_name": (C, [P, I, P, P]),
            "tpfm_set_weight": (I, [P, C, P, I64, I]),
            "tpfm_load_gguf": (I, [P, C, P, ctypes.c_size_t]),
            "tpfm_prepare": (I, [P]),
            "tpfm_forward": (I, [P, P, P, ctypes.c_float, P]),
            "tpfm_sample_chunk": (I, [P, P, P, P, P, I, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_symbols():
    """Function names declared in include/tpmd.h."""
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"\b(tpm[de]_[a-z0-9_]+)\s*\(", txt)))


def _ptr(t):
    """device pointer of a torch tensor (or None)"""
    if t is None:
        return None
    assert t.is_contiguous(), "tensors passed to the library must be contiguous"
    return ctypes.c_void_p(t.data_ptr())


def _hptr(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _stream(stream):
    """a hipStream_t for the C ABI: the given torch stream / handle, else
    torch's current stream (so launches are ordered with torch's copies)"""
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


class MotionDecoder:
    """The decoder context (tpmd_ctx)."""

    def __init__(self, ftype="f32", n_stages=7, ic=None, oc=None, device=0):
        L = lib()
        self.ftype = ftype
        self.n_stages = n_stages
        if ic is not None:
            self._ic = (ctypes.c_int * n_stages)(*ic)
            self._oc = (ctypes.c_int * n_stages)(*oc)
            self.ic, self.oc = tuple(ic), tuple(oc)
        else:
            self._ic = self._oc = None
            self.ic = (512, 512, 512, 512, 256, 128, 64)[:n_stages]
            self.oc = (512, 512, 512, 256, 128, 64, 32)[:n_stages]
        h = L.tpmd_create(device, ftype.encode(), n_stages,
                          ctypes.cast(self._ic, ctypes.c_void_p) if self._ic else None,
                          ctypes.cast(self._oc, ctypes.c_void_p) if self._oc else None)
        if not h:
            raise TpmdError("tpmd_create failed (see stderr)")
        self.h = ctypes.c_void_p(h)
        self.batch = 0
        self.res = 8 << (n_stages - 1)

    def close(self):
        if getattr(self, "h", None):
            lib().tpmd_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != 0:
            raise TpmdError(lib().tpmd_last_error(self.h).decode())
        return rc

    @property
    def last_error(self):
        return lib().tpmd_last_error(self.h).decode()

    # ---- lifecycle
    def set_weight(self, name, arr, f16_file=False, folded=False):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        flags = (W_F16_FILE if f16_file else 0) | (W_FOLDED if folded else 0)
        self._check(lib().tpmd_set_weight(self.h, name.encode(), _hptr(a), a.size, flags))

    def weight_names(self):
        """(name, element count, is_matrix) of every tensor this context expects"""
        out = []
        n, m = ctypes.c_int64(), ctypes.c_int()
        i = 0
        while True:
            nm = lib().tpmd_weight_name(self.h, i, ctypes.byref(n), ctypes.byref(m))
            if nm is None:
                return out
            out.append((nm.decode(), n.value, bool(m.value)))
            i += 1

    def load_gguf(self, path):
        """every decoder tensor of a motion_ae GGUF file (tpmd_load_gguf)"""
        err = ctypes.create_string_buffer(512)
        if lib().tpmd_load_gguf(self.h, str(path).encode(), err, len(err)) != 0:
            raise TpmdError(err.value.decode())

    def set_weights(self, raw):
        for name, (arr, f16) in raw.items():
            self.set_weight(name, arr, f16_file=f16)

    def prepare(self):
        self._check(lib().tpmd_prepare(self.h))

    def build(self, batch):
        self._check(lib().tpmd_build(self.h, int(batch)))
        self.batch = lib().tpmd_batch(self.h)
        self.res = lib().tpmd_out_res(self.h)

    def set_feats(self, feats):
        arrs = [np.ascontiguousarray(f, dtype=np.float32) for f in feats]
        ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
        self._check(lib().tpmd_set_feats(self.h, ctypes.cast(ptrs, ctypes.c_void_p)))

    def set_feats_device(self, feats):
        """feats: torch cuda tensors, or raw device addresses (MotionEncoder.feats_device)"""
        ptrs = (ctypes.c_void_p * len(feats))(*[f if isinstance(f, int) else f.data_ptr() for f in feats])
        self._check(lib().tpmd_set_feats_device(self.h, ctypes.cast(ptrs, ctypes.c_void_p)))

    # ---- decode
    def decode_batch(self, styles):
        """host (n, 512) float32 -> host (n, 3, R, R) float32 (synchronous)"""
        s = np.ascontiguousarray(styles, dtype=np.float32).reshape(-1, 512)
        n = s.shape[0]
        out = np.empty((n, 3, self.res, self.res), np.float32)
        self._check(lib().tpmd_decode_batch(self.h, _hptr(s), n, _hptr(out), 0))
        return out

    def decode_batch_device(self, styles_dev, imgs_dev):
        """device (n, 512) float32 -> device (n, 3, R, R) float32, asynchronous
        (tpmd_decode_batch's on-device ordering rules; frames complete after
        sync())"""
        import torch
        for t, what in ((styles_dev, "styles"), (imgs_dev, "imgs")):
            if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float32):
                raise TpmdError(f"decode_batch_device: {what} must be a float32 CUDA tensor")
            if not t.is_contiguous():
                raise TpmdError(f"decode_batch_device: {what} must be contiguous")
        if styles_dev.dim() != 2 or styles_dev.shape[1] != 512:
            raise TpmdError("decode_batch_device: styles must be (n, 512)")
        n = styles_dev.shape[0]
        if imgs_dev.numel() < n * 3 * self.res * self.res:
            raise TpmdError(f"decode_batch_device: imgs must hold ({n}, 3, {self.res}, {self.res})")
        self._check(lib().tpmd_decode_batch(self.h, _ptr(styles_dev), n, _ptr(imgs_dev), 1))

    def tap_frame_bytes(self, kind, stage):
        return lib().tpmd_tap_frame_bytes(self.h, kind, stage)

    def set_tap(self, kind, stage, buf):
        """copy the decode chain's buffer `kind` of `stage` into the CUDA
        tensor buf on every later decode_batch (None removes the tap)"""
        nb = buf.numel() * buf.element_size() if buf is not None else 0
        self._check(lib().tpmd_set_tap(self.h, kind, stage, _ptr(buf), nb))

    def decode_frames(self, styles, fmt=FRAME_F32, to_buffer=True, cb=None, out=None):
        """a clip of latents (n, 512) through tpmd_decode_frames: returns the
        frames array (n, 3, R, R) f32 or (n, R, R, 3) u8 when to_buffer, and
        calls cb(index, frame_array) per frame (a truthy return stops).  out:
        a caller's host buffer of that shape and type (a numpy array, or a
        torch CPU tensor, pinned or not) to fill instead"""
        s = np.ascontiguousarray(styles, dtype=np.float32).reshape(-1, 512)
        n, R = s.shape[0], self.res
        shape, dt = ((3, R, R), np.float32) if fmt == FRAME_F32 else ((R, R, 3), np.uint8)
        if out is not None:
            nb = out.numel() * out.element_size() if hasattr(out, "numel") else out.nbytes
            if nb != n * int(np.prod(shape)) * np.dtype(dt).itemsize:
                raise TpmdError("decode_frames: out has the wrong size")
            optr = out.data_ptr() if hasattr(out, "data_ptr") else _hptr(out)
        else:
            out = np.empty((n,) + shape, dt) if to_buffer else None
            optr = _hptr(out) if out is not None else None
        nbytes = int(np.prod(shape)) * np.dtype(dt).itemsize

        def tramp(idx, ptr, ud):
            buf = (ctypes.c_char * nbytes).from_address(ptr)
            return 1 if cb(idx, np.frombuffer(buf, dt).reshape(shape).copy()) else 0
        c_cb = FRAME_CB(tramp) if cb else None
        rc = lib().tpmd_decode_frames(self.h, _hptr(s), n, fmt, optr,
                                      ctypes.cast(c_cb, ctypes.c_void_p) if c_cb else None, None)
        if rc < 0:
            raise TpmdError(self.last_error)
        return out

    def decode(self, style):
        s = np.ascontiguousarray(style, dtype=np.float32).reshape(512)
        out = np.empty((3, self.res, self.res), np.float32)
        self._check(lib().tpmd_decode(self.h, _hptr(s), _hptr(out)))
        return out

    def decode_taps(self, style):
        """the reference's tap plan for one latent (tpmd_decode_taps): the
        frame (3, R, R) and {tap name: float32 array in its torch shape}"""
        s = np.ascontiguousarray(style, dtype=np.float32).reshape(512)
        img = np.empty((3, self.res, self.res), np.float32)
        taps = {}

        def put(name, data, ndim, shape, ud):
            sh = tuple(shape[i] for i in range(ndim))
            n = int(np.prod(sh))
            buf = (ctypes.c_float * n).from_address(data)
            taps[name.decode()] = np.frombuffer(buf, np.float32).reshape(sh).copy()
            return 0
        cb = TAP_CB(put)
        self._check(lib().tpmd_decode_taps(self.h, _hptr(s), _hptr(img), ctypes.cast(cb, ctypes.c_void_p), None))
        return img, taps

    def sync(self):
        self._check(lib().tpmd_sync(self.h))

    def use_stream(self, stream=None):
        """enqueue the decoder's work on `stream` (torch stream or handle;
        None = torch's current stream)"""
        self._check(lib().tpmd_set_stream(self.h, _stream(stream)))

    def use_graphs(self, enable=True):
        """replay each lane's launch chain as a HIP graph (default) or
        enqueue its launches one by one"""
        self._check(lib().tpmd_set_graphs(self.h, 1 if enable else 0))

    def profile_stages(self, enable=True):
        return lib().tpmd_profile_stages(self.h, 1 if enable else 0)

    def stage_times(self):
        buf = (ctypes.c_float * 64)()
        n = lib().tpmd_stage_times(self.h, buf, 64)
        return list(buf[:max(n, 0)])

    # ---- per-stage entry points (torch cuda tensors)
    def modconv(self, conv, x, s, y, stream=None):
        n, H, W, _ = x.shape
        self._check(lib().tpmd_modconv(self.h, conv, _ptr(x), n, H, W, _ptr(s), _ptr(y), _stream(stream)))

    def modconv_static(self, conv, x, s, y, stream=None):
        """modconv on the library's static device scratch (allocates nothing)"""
        n, H, W, _ = x.shape
        self._check(lib().tpmd_modconv_static(self.h, conv, _ptr(x), n, H, W, _ptr(s), _ptr(y),
                                              _stream(stream)))

    def stage_tail(self, j, out, s_flow, flow_prev, rgb_prev, flow, trunk, rgb, warp, stream=None):
        n = out.shape[0]
        self._check(lib().tpmd_stage_tail(self.h, j, _ptr(out), n, _ptr(s_flow), _ptr(flow_prev),
                                          _ptr(rgb_prev), _ptr(flow), _ptr(trunk), _ptr(rgb),
                                          _ptr(warp), _stream(stream)))

    def stage_conv_tail(self, j, c1, s_conv, s_flow, flow_prev, rgb_prev, flow, trunk, rgb, warp,
                        stream=None):
        n = c1.shape[0]
        self._check(lib().tpmd_stage_conv_tail(self.h, j, _ptr(c1), n, _ptr(s_conv), _ptr(s_flow),
                                               _ptr(flow_prev), _ptr(rgb_prev), _ptr(flow), _ptr(trunk),
                                               _ptr(rgb), _ptr(warp), _stream(stream)))


def gguf_read_tensor(path, name):
    """(float32 array, stored_as_f16) of one tensor of a GGUF file (no device)"""
    err = ctypes.create_string_buffer(512)
    f16 = ctypes.c_int()
    n = lib().tpmd_gguf_read_tensor(str(path).encode(), name.encode(), None, 0, ctypes.byref(f16), err,
                                    len(err))
    if n < 0:
        raise TpmdError(err.value.decode())
    out = np.empty(n, np.float32)
    if lib().tpmd_gguf_read_tensor(str(path).encode(), name.encode(), _hptr(out), n, ctypes.byref(f16), err,
                                   len(err)) < 0:
        raise TpmdError(err.value.decode())
    return out, bool(f16.value)


# ---- op level (torch cuda tensors)

def gather(feat, W, H, grid, planar=False, sp=False, out=None, stream=None):
    """GGML_OP_BILINEAR_GATHER: feat (W*H, C) f32/f16, grid (N, 2) or planar (2, N)."""
    import torch
    C = feat.shape[-1]
    N = grid.numel() // 2
    if out is None:
        out = torch.empty((C, N) if sp else (N, C), dtype=torch.float32, device=feat.device)
    f16 = feat.dtype == torch.float16
    rc = lib().tpmd_gather(_ptr(feat), int(f16), C, W, H, _ptr(grid), N, int(planar), int(sp),
                           _ptr(out), _stream(stream))
    if rc != 0:
        raise TpmdError("tpmd_gather: invalid arguments")
    return out


def gather_taps(grid, W, H, planar=False, stream=None):
    import torch
    N = grid.numel() // 2
    dev = grid.device
    x0 = torch.empty(N, dtype=torch.int32, device=dev)
    y0 = torch.empty(N, dtype=torch.int32, device=dev)
    wx = torch.empty(N, dtype=torch.float32, device=dev)
    wy = torch.empty(N, dtype=torch.float32, device=dev)
    rc = lib().tpmd_gather_taps(_ptr(grid), W, H, N, int(planar), _ptr(x0), _ptr(y0), _ptr(wx),
                                _ptr(wy), _stream(stream))
    if rc != 0:
        raise TpmdError("tpmd_gather_taps: invalid arguments")
    return x0, y0, wx, wy


def frames_to_rgb24(chw, stream=None):
    """(n, 3, R, R) f32 cuda frames -> (n, R, R, 3) uint8 (the video writer's rule)"""
    import torch
    n, _, R, _ = chw.shape
    rgb = torch.empty((n, R, R, 3), dtype=torch.uint8, device=chw.device)
    if lib().tpmd_frames_to_rgb24(_ptr(chw), n, R, _ptr(rgb), _stream(stream)) != 0:
        raise TpmdError("tpmd_frames_to_rgb24: invalid arguments")
    return rgb


def upfirdn2x(x, k4, stream=None):
    import torch
    H, W = x.shape[-2:]
    CB = x.numel() // (H * W)
    y = torch.empty(x.shape[:-2] + (2 * H, 2 * W), dtype=torch.float32, device=x.device)
    rc = lib().tpmd_upfirdn2x(_ptr(x), _ptr(k4), _ptr(y), W, H, CB, _stream(stream))
    if rc != 0:
        raise TpmdError("tpmd_upfirdn2x: invalid arguments")
    return y


def flow_grid(fl, xs, stream=None):
    import torch
    N = fl.numel() // 3
    y = torch.empty((3, N), dtype=torch.float32, device=fl.device)
    rc = lib().tpmd_flow_grid(_ptr(fl), _ptr(xs), _ptr(y), N, _stream(stream))
    if rc != 0:
        raise TpmdError("tpmd_flow_grid: invalid arguments")
    return y


def probe_mfma_f16(random_operands=True, iters=2000):
    """(TFLOP/s, core GHz) of back-to-back f16 MFMAs on every SIMD with zero
    or random operands (tpmd_probe_mfma_f16)"""
    tf, ghz = ctypes.c_float(), ctypes.c_float()
    rc = lib().tpmd_probe_mfma_f16(1 if random_operands else 0, iters, ctypes.byref(tf), ctypes.byref(ghz))
    if rc != 0:
        raise TpmdError("tpmd_probe_mfma_f16 failed")
    return float(tf.value), float(ghz.value)


class MotionEncoder:
    """tp::motion_enc (src/motion_enc.h:20-30) over tpme_*: run an image,
    read appearance / lambda / motion and the decoder feats.

        enc = MotionEncoder("f16"); enc.set_weights(raw); enc.prepare()
        out = enc.run(image)                 # dict of numpy arrays
        dec.set_feats_device(enc.feats_device())
    """

    def __init__(self, ftype="f32", ch_in=None, ch_out=None, device=0):
        L = lib()
        self.ftype = ftype
        nb = 7 if ch_in is None else len(ch_in)
        self.ch_in = tuple(ch_in) if ch_in is not None else (32, 64, 128, 256, 512, 512, 512)
        self.ch_out = tuple(ch_out) if ch_out is not None else (64, 128, 256, 512, 512, 512, 512)
        self.n_blocks = nb
        a = (ctypes.c_int * nb)(*self.ch_in) if ch_in is not None else None
        b = (ctypes.c_int * nb)(*self.ch_out) if ch_out is not None else None
        h = L.tpme_create(device, ftype.encode(), nb, a, b)
        if not h:
            raise TpmdError("tpme_create failed")
        self.h = h
        self.res = 4 << nb

    def _check(self, rc):
        if rc < 0:
            raise TpmdError(lib().tpme_last_error(self.h).decode())
        return rc

    def close(self):
        if getattr(self, "h", None):
            lib().tpme_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_names(self):
        out, i = [], 0
        n = ctypes.c_int64()
        while True:
            nm = lib().tpme_weight_name(self.h, i, ctypes.byref(n), None)
            if nm is None:
                return out
            out.append((nm.decode(), n.value))
            i += 1

    def set_weights(self, raw, folded=False):
        """raw: name -> (array in torch shape, f16_in_file)"""
        for name, _ in self.weight_names():
            arr, f16 = raw[name]
            a = np.ascontiguousarray(arr, dtype=np.float32)
            flags = (W_F16_FILE if f16 else 0) | (W_FOLDED if folded else 0)
            self._check(lib().tpme_set_weight(self.h, name.encode(), _hptr(a), a.size, flags))

    def load_gguf(self, path):
        """every encoder tensor of a motion_ae GGUF file (tpme_load_gguf)"""
        err = ctypes.create_string_buffer(512)
        if lib().tpme_load_gguf(self.h, str(path).encode(), err, len(err)) < 0:
            raise TpmdError(err.value.decode())

    def prepare(self):
        self._check(lib().tpme_prepare(self.h))

    def run(self, image):
        """image (3, R, R) f32 numpy (host) or torch cuda tensor -> dict with
        appearance, lambda, motion and feats (list of (r*r, C) numpy)"""
        if hasattr(image, "is_cuda") and image.is_cuda:
            self._check(lib().tpme_run(self.h, _ptr(image), 1))
        else:
            im = np.ascontiguousarray(image, dtype=np.float32)
            assert im.shape == (3, self.res, self.res)
            self._check(lib().tpme_run(self.h, _hptr(im), 0))
        app = np.empty(512, np.float32)
        lam = np.empty(20, np.float32)
        mot = np.empty(512, np.float32)
        self._check(lib().tpme_result(self.h, _hptr(app), _hptr(lam), _hptr(mot)))
        return {"appearance": app, "lambda": lam, "motion": mot,
                "feats": [self.level(self.n_blocks - 1 - j) for j in range(self.n_blocks)]}

    def level(self, l):
        """pyramid level l (menc.conv<l>) as (r*r, C) numpy"""
        n = self._check(lib().tpme_level(self.h, l, None))
        out = np.empty(n, np.float32)
        self._check(lib().tpme_level(self.h, l, _hptr(out)))
        r = self.res >> l
        return out.reshape(r * r, -1)

    def feats_device(self):
        """device pointers of the last run's feats j = 0 .. n_blocks-1"""
        ptrs = []
        for j in range(self.n_blocks):
            p = lib().tpme_feat(self.h, j, None, None)
            if not p:
                raise TpmdError("encoder has not run")
            ptrs.append(p)
        return ptrs


class FmtConfig(ctypes.Structure):
    """tpfm_config (include/tpmd.h), fmt_model's hyper-parameters"""
    _fields_ = [(n, ctypes.c_int) for n in ("dim_h", "depth", "n_heads", "dim_w", "dim_a", "dim_e",
                                            "chunk_frames", "prev_frames", "attn_window", "t_freq_dim", "nfe")] + \
               [(n, ctypes.c_float) for n in ("mlp_ratio", "ln_eps", "a_cfg", "e_cfg", "r_cfg")]

    @classmethod
    def default(cls, **kw):
        c = cls()
        lib().tpfm_default_config(ctypes.byref(c))
        for k, v in kw.items():
            setattr(c, k, v)
        return c

    @classmethod
    def from_gguf(cls, path):
        c = cls()
        err = ctypes.create_string_buffer(512)
        if lib().tpfm_read_config(str(path).encode(), ctypes.byref(c), err, len(err)) < 0:
            raise TpmdError(err.value.decode())
        return c

    @property
    def total(self):
        return self.chunk_frames + self.prev_frames


class FlowTransformer:
    """tp::fmt_model (src/fmt.h:9-36) over tpfm_*: forward and sample_chunk"""

    def __init__(self, ftype="f32", cfg=None, device=0):
        self.cfg = cfg if cfg is not None else FmtConfig.default()
        h = lib().tpfm_create(device, ftype.encode(), ctypes.byref(self.cfg))
        if not h:
            raise TpmdError("tpfm_create failed")
        self.h = h
        self.ftype = ftype

    def _check(self, rc):
        if rc < 0:
            raise TpmdError(lib().tpfm_last_error(self.h).decode())
        return rc

    def close(self):
        if getattr(self, "h", None):
            lib().tpfm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_names(self):
        out, i = [], 0
        n = ctypes.c_int64()
        while True:
            nm = lib().tpfm_weight_name(self.h, i, ctypes.byref(n), None)
            if nm is None:
                return out
            out.append((nm.decode(), n.value))
            i += 1

    def set_weights(self, raw):
        for name, _ in self.weight_names():
            arr, f16 = raw[name]
            a = np.ascontiguousarray(arr, dtype=np.float32)
            self._check(lib().tpfm_set_weight(self.h, name.encode(), _hptr(a), a.size, W_F16_FILE if f16 else 0))

    def load_gguf(self, path):
        err = ctypes.create_string_buffer(512)
        if lib().tpfm_load_gguf(self.h, str(path).encode(), err, len(err)) < 0:
            raise TpmdError(err.value.decode())

    def prepare(self):
        self._check(lib().tpfm_prepare(self.h))

    def forward(self, x60, cond, t):
        c = self.cfg
        x = np.ascontiguousarray(x60, dtype=np.float32).reshape(c.total, c.dim_w)
        cd = np.ascontiguousarray(cond, dtype=np.float32).reshape(3, c.total, c.dim_w + c.dim_a + c.dim_e)
        v = np.empty((3, c.total, c.dim_w), np.float32)
        self._check(lib().tpfm_forward(self.h, _hptr(x), _hptr(cd), float(t), _hptr(v)))
        return v

    def sample_chunk(self, wr, prev_x, prev_wa, cond_audio, emotion, x0):
        c = self.cfg
        a = [np.ascontiguousarray(v, dtype=np.float32) for v in (wr, prev_x, prev_wa, cond_audio, x0)]
        out = np.empty((c.chunk_frames, c.dim_w), np.float32)
        self._check(lib().tpfm_sample_chunk(self.h, _hptr(a[0]), _hptr(a[1]), _hptr(a[2]), _hptr(a[3]), int(emotion),
                                            _hptr(a[4]), _hptr(out)))
        return out
