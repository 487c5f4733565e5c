"""Comparison metrics used by the parity tests."""
import numpy as np


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = np.linalg.norm(want.ravel())
    return float(np.linalg.norm((got - want).ravel()) / (d if d > 0 else 1.0))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def _gauss(n=11, sigma=1.5):
    x = np.arange(n) - (n - 1) / 2
    g = np.exp(-x * x / (2 * sigma * sigma))
    return g / g.sum()


def _filt(img, g):
    # separable 'valid' gaussian filter over the last two axes
    from numpy.lib.stride_tricks import sliding_window_view
    n = g.size
    t = sliding_window_view(img, n, axis=-1) @ g
    t = np.swapaxes(sliding_window_view(np.swapaxes(t, -1, -2), n, axis=-1) @ g, -1, -2)
    return t


def ssim(a, b, data_range=None):
    """mean SSIM (Wang et al. 2004, 11x11 gaussian sigma 1.5) over a CHW image"""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if data_range is None:
        data_range = max(b.max() - b.min(), 1e-12)
    c1, c2 = (0.01 * data_range) ** 2, (0.03 * data_range) ** 2
    g = _gauss()
    mu_a, mu_b = _filt(a, g), _filt(b, g)
    saa = _filt(a * a, g) - mu_a ** 2
    sbb = _filt(b * b, g) - mu_b ** 2
    sab = _filt(a * b, g) - mu_a * mu_b
    s = ((2 * mu_a * mu_b + c1) * (2 * sab + c2)) / ((mu_a ** 2 + mu_b ** 2 + c1) * (saa + sbb + c2))
    return float(s.mean())


def to_sp(t, r):
    """a decoder tap as (B, C, r, r): channel-last (B, r*r, C) taps are
    transposed, spatial ones returned as is"""
    t = np.asarray(t)
    if t.ndim == 3 and t.shape[1] == r * r:
        return np.ascontiguousarray(t.reshape(t.shape[0], r, r, -1).transpose(0, 3, 1, 2))
    return t
