"""Whole-decoder GPU parity through the C ABI against the CPU oracle's fast
graph (well-conditioned "smooth" workload; see synth.WORKLOADS):
f32 frames rel-L2 <= 1e-4; f16 frames SSIM >= 0.99 and cosine >= 0.999."""
import numpy as np
import pytest

import synth
import tpmd
from metrics import cosine, rel_l2, ssim

pytestmark = pytest.mark.gpu

SMALL_IC = (64, 64, 64, 64, 32, 32, 32)
SMALL_OC = (64, 64, 64, 32, 32, 32, 32)


def _decoders(om, ftype, ic, oc, nf, batch, workload="smooth"):
    raw, lat, feats = synth.workload(workload, nf, ftype, ic, oc)
    ref = om.Decoder(raw, ftype, ic, oc)
    ref.set_feats(feats)
    dec = tpmd.MotionDecoder(ftype, len(ic), ic, oc)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(batch)
    dec.set_feats(feats)
    return ref, dec, lat


def _frame_ok(ftype, got, want):
    if ftype == "f32":
        assert rel_l2(got, want) <= 1e-4, rel_l2(got, want)
    else:
        c, s = cosine(got, want), ssim(got, want)
        assert c >= 0.999 and s >= 0.99, (c, s)


@pytest.mark.parametrize("ftype", ["f32", "f16"])
def test_decoder_small(om, torch_cuda, ftype):
    ref, dec, lat = _decoders(om, ftype, SMALL_IC, SMALL_OC, 3, 4)
    want = ref.decode_fast(lat)
    got = dec.decode_batch(lat)          # n = 3 < batch = 4
    assert got.shape == (3, 3, 512, 512)
    for b in range(3):
        _frame_ok(ftype, got[b], want[b])


@pytest.mark.parametrize("ftype", ["f16", "f32"])
def test_decoder_reference_channels(om, torch_cuda, ftype):
    ref, dec, lat = _decoders(om, ftype, synth.REF_IC, synth.REF_OC, 2, 2)
    want = ref.decode_fast(lat)
    got = dec.decode_batch(lat)
    for b in range(2):
        _frame_ok(ftype, got[b], want[b])


def test_decode_paths_agree(om, torch_cuda):
    """decode (one frame), decode_batch (host) and the device path agree bit
    for bit, and a frame does not depend on its batch neighbours"""
    torch = torch_cuda
    _, dec, lat = _decoders(om, "f16", SMALL_IC, SMALL_OC, 3, 3)
    full = dec.decode_batch(lat)
    one = dec.decode(lat[1])
    assert np.array_equal(one, full[1])
    part = dec.decode_batch(lat[1:])
    assert np.array_equal(part, full[1:])
    sd = torch.from_numpy(lat).cuda()
    out = torch.empty((3, 3, 512, 512), device="cuda")
    dec.use_stream()                     # order the decode after torch's copy
    dec.decode_batch_device(sd, out)
    dec.sync()
    assert np.array_equal(out.cpu().numpy(), full)


def test_multi_lane_device_decodes(om, torch_cuda):
    """device decodes on the library's own stream rotate over the decoder's
    lanes (consecutive batches overlap on the GPU; four batches reach every
    lane and reuse the first): every batch equals the host path bit for bit,
    the ragged last one included"""
    torch = torch_cuda
    _, dec, lat = _decoders(om, "f16", SMALL_IC, SMALL_OC, 7, 2)
    starts = range(0, 7, 2)
    want = np.concatenate([dec.decode_batch(lat[t:t + 2]) for t in starts])
    sd = torch.from_numpy(lat).cuda()
    outs = [torch.empty((min(2, 7 - t), 3, 512, 512), device="cuda") for t in starts]
    torch.cuda.synchronize()             # inputs ready before the decoder's streams read them
    for o, t in zip(outs, starts):
        dec.decode_batch_device(sd[t:t + 2], o)
    dec.sync()
    assert np.array_equal(np.concatenate([o.cpu().numpy() for o in outs]), want)


def test_error_contract(torch_cuda):
    dec = tpmd.MotionDecoder("f32", 2, (64, 64), (64, 64))
    with pytest.raises(tpmd.TpmdError, match="decoder not prepared"):
        dec.build(2)
    with pytest.raises(tpmd.TpmdError, match="missing tensor"):
        dec.prepare()
    with pytest.raises(tpmd.TpmdError, match="unknown decoder tensor"):
        dec.set_weight("dec.nope", np.zeros(4, np.float32))
    with pytest.raises(tpmd.TpmdError, match="elements"):
        dec.set_weight("dec.conv1.activate.bias", np.zeros(5, np.float32))
    raw = synth.raw_weights(1000, "f32", (64, 64), (64, 64))
    dec.set_weights(raw)
    dec.prepare()
    with pytest.raises(tpmd.TpmdError, match="decoder not built"):
        dec.set_feats(synth.feats(1002, (64, 64)))
    dec.build(2)
    with pytest.raises(tpmd.TpmdError, match="feats not set"):
        dec.decode_batch(np.zeros((1, 512), np.float32))
    dec.set_feats(synth.feats(1002, (64, 64)))
    with pytest.raises(tpmd.TpmdError, match="1..2 styles"):
        dec.decode_batch(np.zeros((3, 512), np.float32))
    assert tpmd.MotionDecoder.__init__  # constructor rejects bad configs:
    with pytest.raises(tpmd.TpmdError):
        tpmd.MotionDecoder("f32", 2, (64, 48), (48, 64))


def test_lanes_read_latents_in_order(om, torch_cuda):
    """one latent buffer refilled on torch's default stream (HIP's null
    stream) right after each device decode, with no synchronisation: every
    call decodes the latents it was given (a call reads them after earlier
    null-stream work, and later null-stream work waits for that read)"""
    torch = torch_cuda
    assert torch.cuda.current_stream().cuda_stream == 0, "torch's current stream is not the null stream"
    _, dec, lat = _decoders(om, "f16", SMALL_IC, SMALL_OC, 8, 2)
    starts = range(0, 8, 2)
    want = [dec.decode_batch(lat[t:t + 2]) for t in starts]
    src = torch.from_numpy(lat).cuda()
    sd = torch.empty((2, 512), device="cuda")
    outs = [torch.empty((2, 3, 512, 512), device="cuda") for _ in starts]
    torch.cuda.synchronize()
    for o, t in zip(outs, starts):
        sd.copy_(src[t:t + 2])
        dec.decode_batch_device(sd, o)
    dec.sync()
    for o, w in zip(outs, want):
        assert np.array_equal(o.cpu().numpy(), w)


def test_lanes_reuse_one_frame_buffer(om, torch_cuda):
    """four device decodes into one frame buffer (every lane, then lane 0
    again, the calls overlapping on the GPU): after tpmd_sync it holds the
    last call's frames; a buffer that only partly overlaps the previous
    call's is ordered too"""
    torch = torch_cuda
    _, dec, lat = _decoders(om, "f16", SMALL_IC, SMALL_OC, 8, 2)
    want = dec.decode_batch(lat[6:8])
    src = torch.from_numpy(lat).cuda()
    out = torch.empty((3, 3, 512, 512), device="cuda")
    torch.cuda.synchronize()
    for t in range(0, 8, 2):
        dec.decode_batch_device(src[t:t + 2], out[:2])
    dec.sync()
    assert np.array_equal(out[:2].cpu().numpy(), want)
    # frames 1..2 of the buffer after frames 0..1: the shared frame holds the later call's
    dec.decode_batch_device(src[0:2], out[0:2])
    dec.decode_batch_device(src[6:8], out[1:3])
    dec.sync()
    assert np.array_equal(out[1:3].cpu().numpy(), want)
