"""The FMT oracle (oracle/fmt.py, the reference's graph, src/fmt.cpp:44-205)
against the upstream torch formulation (tests/fmt_torch.py: F.layer_norm,
scaled_dot_product_attention with a boolean band mask, tanh GELU), plus the
sampler's closed-form pieces (band mask, timestep features, CFG branches)."""
import math

import numpy as np
import pytest

import synth
from metrics import rel_l2

torch = pytest.importorskip("torch")
import fmt_torch  # noqa: E402


def small(OF):
    return OF.Config(dim_h=128, depth=2, n_heads=4, dim_w=64, dim_a=64, chunk_frames=12, prev_frames=4,
                     t_freq_dim=32, nfe=4)


def test_band_mask_and_tfreq(oracle_fmt):
    m = oracle_fmt.band_mask(60, 2)
    assert (m == 0).sum() == 60 * 5 - 2 * (2 + 1)           # rows clipped at both ends
    assert m[10, 8] == 0 and m[10, 12] == 0 and np.isneginf(m[10, 13]) and np.isneginf(m[10, 7])
    tf = oracle_fmt.t_freq(0.0, 256)
    assert np.array_equal(tf[:128], np.ones(128, np.float32)) and np.array_equal(tf[128:], np.zeros(128, np.float32))
    tf = oracle_fmt.t_freq(0.5, 8)
    want = [math.cos(0.5 * math.exp(-math.log(1e4) * k / 4)) for k in range(4)]
    assert np.allclose(tf[:4], want, rtol=1e-6)


@pytest.mark.parametrize("t", [0.0, 0.37, 1.0])
def test_forward_matches_upstream(oracle_fmt, t):
    cfg = small(oracle_fmt)
    raw = synth.fmt_raw_weights(cfg)
    g = np.random.default_rng(3)
    x60 = g.standard_normal((cfg.total, cfg.dim_w)).astype(np.float32)
    cond = g.standard_normal((3, cfg.total, cfg.dim_c)).astype(np.float32)
    got = oracle_fmt.FMT(raw, cfg).forward(x60, cond, t)
    want = fmt_torch.forward(raw, cfg, x60, cond, t)
    assert got.shape == (3, cfg.total, cfg.dim_w)
    assert rel_l2(got, want) <= 1e-5


def test_cond_rows_branches(oracle_fmt):
    cfg = small(oracle_fmt)
    F = oracle_fmt.FMT(synth.fmt_raw_weights(cfg), cfg)
    io = synth.fmt_chunk_inputs(cfg)
    c = F.cond_rows(io["wr"], io["prev_wa"], io["cond_audio"], 3)
    D, A, P = cfg.dim_w, cfg.dim_a, cfg.prev_frames
    assert np.array_equal(c[:, :, :D], np.broadcast_to(io["wr"], (3, cfg.total, D)))
    assert np.array_equal(c[0, :P, D:D + A], io["prev_wa"]) and not c[0, P:, D:D + A].any()
    assert np.array_equal(c[2, P:, D:D + A], io["cond_audio"])
    assert (c[1, :, D + A + 3] == 1).all() and c[1, :, D + A:].sum() == cfg.total
    assert not c[0, :, D + A:].any() and not c[2, :, D + A:].any()


def test_sampler_is_euler_with_cfg(oracle_fmt):
    """nfe = 2: one Euler step of the CFG-combined velocity from t = 0"""
    cfg = oracle_fmt.Config(dim_h=64, depth=1, n_heads=2, dim_w=32, dim_a=32, chunk_frames=6, prev_frames=2,
                            t_freq_dim=16, nfe=2)
    F = oracle_fmt.FMT(synth.fmt_raw_weights(cfg), cfg)
    io = synth.fmt_chunk_inputs(cfg)
    x = F.sample_chunk(io["wr"], io["prev_x"], io["prev_wa"], io["cond_audio"], 1, io["x0"])
    cond = F.cond_rows(io["wr"], io["prev_wa"], io["cond_audio"], 1)
    v = F.forward(np.concatenate([io["prev_x"], io["x0"]]), cond, 0.0)
    vc = (v[0] + 2.0 * (v[2] - v[0])) + 1.0 * (v[1] - v[2])
    assert np.allclose(x, io["x0"] + vc[2:], rtol=1e-5, atol=1e-5)


def test_tensor_list_matches_synth(oracle_fmt):
    """the oracle's FMT tensor inventory and the synthetic-weight generator's
    (two independent restatements of src/fmt.cpp:61-150) agree"""
    for kw in ({}, dict(dim_h=128, depth=2, n_heads=4, dim_w=64, dim_a=64)):
        cfg = oracle_fmt.Config(**kw)
        assert oracle_fmt.weight_names(cfg) == synth.fmt_tensor_shapes(cfg)
        assert oracle_fmt.weight_names(cfg) == synth.fmt_tensor_shapes(synth.FmtConfig(**kw))
