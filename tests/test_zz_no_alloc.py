"""tpmd_modconv_static, the entry point that allocates nothing (its scratch
is the library's static per-GPU device array), against tpmd_modconv through
the C ABI: the same kernels on the same inputs, so the outputs agree bit for
bit, on two calls in a row whose second is smaller (it runs split-K, so its
partial sums also live in the static scratch); a call needing more scratch
than the array holds is refused."""
import numpy as np
import pytest

import synth
import tpmd

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ftype", ["f16", "f32"])
def test_modconv_static_matches_modconv(torch_cuda, ftype):
    torch = torch_cuda
    dec = tpmd.MotionDecoder(ftype, 7)
    dec.set_weights(synth.raw_weights(1000, ftype))
    dec.prepare()
    g = torch.Generator(device="cuda").manual_seed(5)
    # (conv, frames, input side, IC, OC): stage 3's up-conv (512 -> 256 at
    # 32x32 input), then stage 1's (512 -> 512 at 8x8, split-K)
    for conv, n, H, IC, OC in ((7, 3, 32, 512, 256), (3, 2, 8, 512, 512)):
        x = torch.randn((n, H, H, IC), device="cuda", generator=g)
        s = torch.randn((n, IC), device="cuda", generator=g)
        want = torch.empty((n, 2 * H, 2 * H, OC), device="cuda")
        got = torch.full_like(want, float("nan"))
        dec.modconv(conv, x, s, want)
        dec.modconv_static(conv, x, s, got)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (ftype, conv)
    # stage 6's up-conv on 4 frames of 256x256 needs 32 MiB (f16) of scratch
    x = torch.zeros((4, 256, 256, 64), device="cuda")
    s = torch.ones((4, 64), device="cuda")
    y = torch.empty((4, 512, 512, 32), device="cuda")
    with pytest.raises(tpmd.TpmdError, match="bytes of scratch"):
        dec.modconv_static(13, x, s, y)
    dec.close()
