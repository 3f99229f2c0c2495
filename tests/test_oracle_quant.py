"""Pin the absmax/448 quantizers by their invariants."""
import numpy as np

from oracle import formats as F
from oracle import quant as Q


def _half_ulp(v):
    """Half the e4m3 spacing at |v| (v already on the e4m3 grid)."""
    a = np.abs(v)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -6)))
    return 0.5 * 2.0 ** (e - 3)


def test_act_quant_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 512)).astype(np.float32)
    x[3, 128:256] = 0.0                                   # all-zero block -> amax floor
    q, s = Q.quant_act_1x128(x)
    assert s.shape == (7, 4) and np.all(s > 0)
    v = F.e4m3_to_f32(q).reshape(7, 4, 128)
    assert not np.isnan(v).any()
    amax = np.abs(v).max(axis=2)
    nz = np.abs(x.reshape(7, 4, 128)).max(axis=2) > 1e-4
    assert np.all(amax[nz] == 448.0)
    recon = v * s[:, :, None]
    err = np.abs(recon - x.reshape(7, 4, 128))
    xs = np.abs(x.reshape(7, 4, 128) / s[:, :, None])
    assert np.all(err <= (_half_ulp(xs) * 1.0001 + 2.0 ** -10) * s[:, :, None])
    assert np.all(q[3, 128:256] == 0)


def test_weight_quant_invariants():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((256, 384)).astype(np.float32) * 0.02
    q, s = Q.quant_weight_128x128(w)
    assert s.shape == (2, 3)
    v = F.e4m3_to_f32(q).reshape(2, 128, 3, 128)
    assert np.all(np.abs(v).max(axis=(1, 3)) == 448.0)
    recon = v * s[:, None, :, None]
    rel = np.abs(recon - w.reshape(2, 128, 3, 128)).max() / np.abs(w).max()
    assert rel < 1 / 16
