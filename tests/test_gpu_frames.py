"""Frame output path (tpmd_decode_frames): a clip decoded in launches of
`batch` frames with the downloads overlapped; frames equal decode_batch's
bit for bit, RGB24 frames equal the video writer's conversion
(tools/tp-cli.cpp:43-53) computed in numpy, and the per-frame callback has
tp_frame_cb semantics (in order, nonzero stops, n_frames returned)."""
import numpy as np
import pytest

import synth
import tpmd

pytestmark = pytest.mark.gpu

IC = (64, 64, 64, 32, 32, 32, 32)
OC = (64, 64, 32, 32, 32, 32, 32)


def to_rgb24(chw):
    """tools/tp-cli.cpp:43-53 in float32: clamp, (v + 1) / 2 * 255, truncate"""
    x = np.clip(chw.astype(np.float32), np.float32(-1), np.float32(1))
    v = (x + np.float32(1)) / np.float32(2) * np.float32(255)
    return np.moveaxis(v.astype(np.uint8), -3, -1)


@pytest.fixture(scope="module")
def dec():
    raw, _, feats = synth.workload("smooth", 1, "f16", IC, OC)
    d = tpmd.MotionDecoder("f16", len(IC), IC, OC)
    d.set_weights(raw)
    d.prepare()
    d.build(4)
    d.set_feats(feats)
    return d


def test_frames_f32_match_decode_batch(torch_cuda, dec):
    lat = synth.latents(11, 1001, "ar1")                 # 3 launches of 4, last one ragged
    got = dec.decode_frames(lat)
    want = np.concatenate([dec.decode_batch(lat[t:t + 4]) for t in range(0, 11, 4)])
    assert np.array_equal(got, want)


def test_frames_rgb24(torch_cuda, dec):
    torch = torch_cuda
    lat = synth.latents(6, 1001, "ar1") * np.float32(3)  # push values past [-1, 1]
    f32 = dec.decode_frames(lat)
    assert (np.abs(f32) > 1).any()
    rgb = dec.decode_frames(lat, tpmd.FRAME_RGB24)
    assert rgb.shape == (6, 512, 512, 3) and rgb.dtype == np.uint8
    assert np.array_equal(rgb, to_rgb24(f32))
    op = tpmd.frames_to_rgb24(torch.from_numpy(f32).cuda()).cpu().numpy()
    assert np.array_equal(op, rgb)


def test_frame_callback_stops(torch_cuda, dec):
    lat = synth.latents(10, 1001, "ar1")
    want = dec.decode_frames(lat)
    seen = []

    def cb(i, frame):
        seen.append(i)
        assert np.array_equal(frame, want[i])
        return i == 5                                    # stop after frame 5
    assert dec.decode_frames(lat, to_buffer=False, cb=cb) is None
    assert seen == list(range(6))
    # the context keeps working after a stopped stream
    assert np.array_equal(dec.decode_frames(lat[:3]), want[:3])


def test_frames_reuse_lanes_and_slots(torch_cuda, dec):
    """more launches than lanes: every lane and frame slot is reused (the
    slot's previous download must finish first), frames unchanged"""
    lat = synth.latents(30, 1002, "ar1")                 # 8 launches of 4, last one ragged
    got = dec.decode_frames(lat)
    want = np.concatenate([dec.decode_batch(lat[t:t + 4]) for t in range(0, 30, 4)])
    assert np.array_equal(got, want)
    rgb = dec.decode_frames(lat, tpmd.FRAME_RGB24)
    assert np.array_equal(rgb, to_rgb24(want))


def test_frames_on_caller_stream(torch_cuda):
    """on a caller's stream every launch runs on lane 0 in that stream"""
    torch = torch_cuda
    raw, _, feats = synth.workload("smooth", 1, "f16", IC, OC)
    d = tpmd.MotionDecoder("f16", len(IC), IC, OC)
    d.set_weights(raw)
    d.prepare()
    d.build(4)
    d.set_feats(feats)
    lat = synth.latents(18, 1003, "ar1")
    want = np.concatenate([d.decode_batch(lat[t:t + 4]) for t in range(0, 18, 4)])
    s = torch.cuda.Stream()
    d.use_stream(s)
    got = d.decode_frames(lat)
    torch.cuda.synchronize()
    assert np.array_equal(got, want)
    d.close()


def test_frames_into_caller_buffers(torch_cuda, dec):
    """a pinned caller buffer takes the downloads directly, a pageable one is
    filled from the pinned staging; both hold decode_batch's frames, and the
    callback sees the same frames"""
    torch = torch_cuda
    lat = synth.latents(14, 1004, "ar1")
    want = np.concatenate([dec.decode_batch(lat[t:t + 4]) for t in range(0, 14, 4)])
    for pinned in (True, False):
        buf = torch.empty((14, 3, 512, 512), dtype=torch.float32, pin_memory=pinned)
        seen = []

        def cb(i, frame):
            seen.append(i)
            assert np.array_equal(frame, want[i])
            return False
        dec.decode_frames(lat, cb=cb, out=buf)
        assert seen == list(range(14))
        assert np.array_equal(buf.numpy(), want)
    rgb = torch.empty((14, 512, 512, 3), dtype=torch.uint8, pin_memory=True)
    dec.decode_frames(lat, tpmd.FRAME_RGB24, out=rgb)
    assert np.array_equal(rgb.numpy(), to_rgb24(want))
