"""The decode chain at the reference widths, exactly as decode_batch runs it
(f16 activations pre-scaled by the next conv's style, the permuted weight
copies, the batch-size-dependent tile choice), graded launch group by launch
group against the oracle (tests/chain_check.py) on the i.i.d. workload:

  * 16 frames per call (the throughput configuration's launch chains),
  * 50 frames per call (one chunk of the f16 chunk configuration),
  * the warp/demod stress configuration (50 frames, flows x8, latents x8 /
    x1/8),

checking the first two, the middle and the last frame of each call (they
cover the first, a full and the ragged last workgroup tile of every launch).
Then: every frame of a 16- and a 50-frame call equals the same latents
decoded 2 frames per call, bit for bit (a frame's result does not depend on
its batch, although the tile configuration does)."""
import numpy as np
import pytest

import chain_check
import synth
import tpmd

pytestmark = pytest.mark.gpu

_DEC = {}


def _decoder(ftype, workload, batch):
    """one decoder per (ftype, workload) at the largest batch any test here
    needs, kept for the module (weights and feats are the slow part)"""
    key = (ftype, workload)
    if key not in _DEC:
        raw, lat, feats = synth.workload(workload, 50, ftype)
        dec = tpmd.MotionDecoder(ftype, 7)
        dec.set_weights(raw)
        dec.prepare()
        dec.build(50)
        dec.set_feats(feats)
        _DEC[key] = (raw, lat, feats, dec)
    return _DEC[key]


@pytest.fixture(scope="module", autouse=True)
def _release():
    yield
    for v in _DEC.values():
        v[3].close()
    _DEC.clear()


def _frames(n):
    return sorted({0, 1, n // 2, n - 1})


@pytest.mark.parametrize("ftype,workload,n", [
    ("f16", "iid", 16), ("f16", "iid", 50), ("f32", "iid", 16), ("f32", "iid", 50),
    ("f16", "stress", 50),
])
def test_chain_stages(om, torch_cuda, ftype, workload, n):
    torch = torch_cuda
    raw, lat, feats, dec = _decoder(ftype, workload, n)
    ref = om.Decoder(raw, ftype)
    ref.set_feats(feats)
    bufs = chain_check.register_taps(torch, dec, n)
    try:
        sd = torch.from_numpy(lat[:n]).cuda()
        imgs = torch.empty((n, 3, 512, 512), device="cuda")
        torch.cuda.synchronize()
        dec.decode_batch_device(sd, imgs)
        dec.sync()
        F = _frames(n)
        rep = chain_check.check_chain(om, ref, bufs, lat[:n], F, imgs[F].cpu().numpy(), ftype)
    finally:
        chain_check.clear_taps(dec, bufs)
    worst = max(rep, key=lambda t: t[1])
    print(f"{ftype} {workload} n={n}: {len(rep)} checks, worst rel-L2 {worst[1]:.2e} at {worst[0]}")


@pytest.mark.parametrize("ftype", ["f16", "f32"])
def test_batch_independent_bits(torch_cuda, ftype):
    torch = torch_cuda
    _, lat, _, dec = _decoder(ftype, "iid", 50)
    sd = torch.from_numpy(lat).cuda()
    torch.cuda.synchronize()
    small = torch.empty((50, 3, 512, 512), device="cuda")
    dec.use_stream()                      # one stream: calls run in order
    for t in range(0, 50, 2):
        dec.decode_batch_device(sd[t:t + 2], small[t:t + 2])
    for n in (16, 50):
        big = torch.empty((n, 3, 512, 512), device="cuda")
        dec.decode_batch_device(sd[:n], big)
        dec.sync()
        same = (big == small[:n]).flatten(1).all(1).cpu().numpy()
        assert same.all(), (ftype, n, np.nonzero(~same)[0].tolist())
        del big


def test_throughput_clip_frames(torch_cuda):
    """the throughput configuration: a 250-frame clip (f16, reference widths)
    through the frame output path in launches of 16 frames rotating over the
    decoder's lanes (the ragged last launch holds 10): every frame equals the
    same latent decoded in a 2-frame call, bit for bit"""
    raw, lat, feats = synth.workload("iid", 250, "f16")
    dec = tpmd.MotionDecoder("f16", 7)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(16)
    dec.set_feats(feats)
    clip = dec.decode_frames(lat, tpmd.FRAME_F32)
    assert clip.shape == (250, 3, 512, 512)
    bad = [t + i for t in range(0, 250, 2)
           for i, f in enumerate(dec.decode_batch(lat[t:t + 2])) if not np.array_equal(f, clip[t + i])]
    dec.close()
    assert not bad, bad[:10]
