"""Pinning of the oracle's MIMO entanglement statistics (tesm_mimo.py:458-523) on the CPU.

The reference's fixtures hold the RoPE'd q and k the statistics are taken on (the arguments of
_compute_local_entanglement_mimo); the checks are a float64 brute force over explicit loops, a
one-hot case whose only nonzero score sits at a known (window, head, slot), and the count identity.
"""
import math

import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from oracle import tesm_torch as ot


def _module(H, R, W, thr):
    torch.manual_seed(0)
    return ot.TESMMIMO_Optimized(d_model=32, d_state=8, n_heads=H, mimo_rank=2, ent_rank=R, entanglement_window=W,
                                 entanglement_threshold=thr, max_seq_len=128).eval()


def _brute(q, k, W, thr):
    """float64 loops: window v covers key positions v..v+W-1 and is queried at position W-1+v."""
    B, L, H, R = q.shape
    S = min(L, 64)
    V = S - W + 1
    out = np.zeros((B, V, H, W))
    sc = np.zeros((B, V, H, W))
    for b in range(B):
        for v in range(V):
            for h in range(H):
                for w in range(W):
                    s = sum(float(q[b, W - 1 + v, h, r]) * float(k[b, v + w, h, r]) for r in range(R)) / math.sqrt(R)
                    sc[b, v, h, w] = s
                    out[b, v, h, w] = 1.0 if s > thr else (-1.0 if s < -thr else 0.0)
    return out, sc


@pytest.mark.parametrize("name", ["mimo_f32", "mimo_f32_w3"])
def test_stats_on_fixture_qk_match_brute_force(name):
    g, meta = load_golden(name), golden_meta(name)
    q = torch.from_numpy(g["_compute_local_entanglement_mimo/arg0#0"])
    k = torch.from_numpy(g["_compute_local_entanglement_mimo/arg1#0"])
    B, L, H, R = q.shape
    W = meta["W"]
    thr = 0.02
    m = _module(H, R, W, thr)
    m._update_entanglement_stats_mimo(q, k)
    want, sc = _brute(q.numpy(), k.numpy(), W, thr)
    got = m._stats_ternary_buffer.reshape(want.shape).numpy()
    clear = np.abs(np.abs(sc) - thr) > 1e-5  # decisions not at the threshold within float32 rounding
    assert np.array_equal(got[clear], want[clear])
    st = m.last_entanglement_stats
    n = want.size
    assert m._ternary_stats_for_logging[1] == float(n)
    assert abs(st["positive"] - (got > 0).sum() / n) < 1e-12
    assert abs(st["negative"] - (got < 0).sum() / n) < 1e-12
    assert abs(st["positive"] + st["negative"] + st["zero"] - 1.0) < 1e-12
    assert 0 < st["positive"] < 1 and 0 < st["negative"] < 1  # the threshold splits these scores


def test_stats_one_hot_position():
    """Only q[W-1+v0, h0] and k[v0+w0, h0] are nonzero: exactly one +1 at (v0, h0, w0)."""
    B, L, H, R, W = 2, 40, 3, 8, 6
    v0, h0, w0 = 7, 1, 4
    q = torch.zeros(B, L, H, R)
    k = torch.zeros(B, L, H, R)
    q[1, W - 1 + v0, h0, 2] = 2.0
    k[1, v0 + w0, h0, 2] = 3.0
    m = _module(H, R, W, 0.5)
    m._update_entanglement_stats_mimo(q, k)
    t = m._stats_ternary_buffer.reshape(B, L - W + 1, H, W)
    assert t.shape == (B, 35, H, W)
    nz = torch.nonzero(t)
    assert nz.tolist() == [[1, v0, h0, w0]]
    assert m.last_entanglement_stats["positive"] == 1.0 / t.numel()
    # negative score for the mirrored key
    k[1, v0 + w0, h0, 2] = -3.0
    m._update_entanglement_stats_mimo(q, k)
    assert m.last_entanglement_stats["negative"] == 1.0 / t.numel()


def test_stats_sample_limits():
    """At most 64 positions are sampled and a window longer than the sample fails as in the reference."""
    q = torch.randn(1, 100, 2, 4)
    k = torch.randn(1, 100, 2, 4)
    m = _module(2, 4, 16, 0.1)
    m._update_entanglement_stats_mimo(q, k)
    assert m._stats_ternary_buffer.numel() == (64 - 16 + 1) * 2 * 16
    m = _module(2, 4, 80, 0.1)
    with pytest.raises(RuntimeError):
        m._update_entanglement_stats_mimo(q, k)
