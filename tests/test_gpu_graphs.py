"""The decode chain replayed as HIP graphs (tpmd_set_graphs, on by default)
against the same chain enqueued launch by launch: every replay's frames equal
the eager frames bit for bit, with the program's own eager GPU work and
synchronisations between replays; the per-lane graph cache (4 per lane)
keyed by frame count and frame buffer, including evictions; and the three
lanes of device-resident decodes."""
import numpy as np
import pytest

import synth
import tpmd

pytestmark = pytest.mark.gpu

IC = (64, 64, 64, 32, 32, 32, 32)
OC = (64, 64, 32, 32, 32, 32, 32)


@pytest.fixture(scope="module")
def dec_and_lat():
    raw, lat, feats = synth.workload("smooth", 16, "f16", IC, OC)
    dec = tpmd.MotionDecoder("f16", len(IC), IC, OC)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(8)
    dec.set_feats(feats)
    yield dec, lat
    dec.close()


def test_graph_replays_match_eager(torch_cuda, dec_and_lat):
    torch = torch_cuda
    dec, lat = dec_and_lat
    dec.use_graphs(False)
    want = {n: dec.decode_batch(lat[:n]) for n in (8, 5, 3)}
    dec.use_graphs(True)
    noise = torch.randn(1 << 20, device="cuda")
    # host-buffer calls run on lane 0: one frame buffer, three frame counts
    for rep in range(3):
        for n in (8, 5, 8, 3):
            got = dec.decode_batch(lat[:n])
            assert np.array_equal(got, want[n]), (rep, n)
            noise.mul_(1.0001).add_(0.5)          # eager work between replays
            torch.cuda.synchronize()


def test_graph_cache_evicts(torch_cuda, dec_and_lat):
    """more (frames, buffer) pairs on one lane than the cache holds"""
    torch = torch_cuda
    dec, lat = dec_and_lat
    R = dec.res
    sd = torch.from_numpy(lat[:8]).cuda()
    dec.use_graphs(False)
    dec.use_stream()                              # every call on lane 0, in order
    want = torch.empty((8, 3, R, R), device="cuda")
    dec.decode_batch_device(sd, want)
    dec.sync()
    dec.use_graphs(True)
    bufs = [torch.empty((8, 3, R, R), device="cuda") for _ in range(6)]
    for rep in range(2):
        for i, b in enumerate(bufs):
            n = 8 - i
            b.fill_(float("nan"))
            dec.decode_batch_device(sd[:n], b)
            dec.sync()
            assert torch.equal(b[:n], want[:n]), (rep, i)


def test_graph_lanes(torch_cuda, dec_and_lat):
    """device-resident decodes on the decoder's own lanes, graphs on and off"""
    torch = torch_cuda
    raw, lat, feats = synth.workload("smooth", 16, "f16", IC, OC)
    dec = tpmd.MotionDecoder("f16", len(IC), IC, OC)
    try:
        dec.set_weights(raw)
        dec.prepare()
        dec.build(8)
        dec.set_feats(feats)
        R = dec.res
        sd = torch.from_numpy(lat).cuda()
        outs = {}
        for graphs in (False, True):
            dec.use_graphs(graphs)
            o = [torch.empty((8, 3, R, R), device="cuda") for _ in range(3)]
            torch.cuda.synchronize()
            for rep in range(4):
                for k in range(6):
                    dec.decode_batch_device(sd[(k % 2) * 8:(k % 2) * 8 + 8], o[k % 3])
            dec.sync()
            outs[graphs] = [x.cpu() for x in o]
        for a, b in zip(outs[False], outs[True]):
            assert torch.equal(a, b)
    finally:
        dec.close()
