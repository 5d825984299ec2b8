"""Pinning of the oracle's global entanglement pieces on the CPU (the reference's SISO global path is
pinned by the siso_global_f32 fixture; these cover what it leaves open).

* _global_rel_bias (tesm.py:970-982): in float32 positions are exact, so the bias is a function of
  i - j alone (Toeplitz) and equals the closed form sum_p e_p (sin + cos)(d * p * pi / 1000) * scale
  + bias; in bf16 the positions are rounded (arange in bf16), which a pair of rows makes visible.
* _global_ent_mimo (tesm_mimo.py:655-687): against a float64 brute force over explicit loops.
"""
import math

import numpy as np
import torch

from oracle import tesm_torch as ot


def _siso(L=64, thr=0.05):
    torch.manual_seed(0)
    m = ot.TESM_SISO(d_model=32, d_state=8, ent_rank=8, entanglement_window=0, entanglement_threshold=thr,
                     max_seq_len=max(L, 64)).eval()
    with torch.no_grad():
        m.global_rel_pos_embed.copy_(torch.randn(m.global_rel_pos_embed.shape, generator=torch.Generator().manual_seed(1)) * 0.05)
        m.global_rel_pos_scale.fill_(1.5)
        m.global_rel_pos_bias.fill_(-0.01)
    return m


def test_rel_bias_f32_is_toeplitz_closed_form():
    m = _siso()
    L = 40
    with torch.no_grad():
        b = m._global_rel_bias(L, torch.float32, "cpu").double().numpy()
    e = m.global_rel_pos_embed.detach().double().numpy()
    P = e.shape[0]
    for i in range(L):
        for j in range(L):
            d = i - j
            ang = d * np.arange(1, P + 1) * math.pi / 1000.0
            want = (np.sum(np.sin(ang) * e) + np.sum(np.cos(ang) * e)) * 1.5 - 0.01
            assert abs(b[i, j] - want) < 1e-5, (i, j)
            assert b[i, j] == b[i - j if i >= j else 0, 0] or i < j  # Toeplitz on the causal side


def test_rel_bias_bf16_uses_rounded_positions():
    """arange(300) in bf16 maps 257 to 256: rows 256 and 257 of the bias are identical."""
    m = _siso(L=300)
    with torch.no_grad():
        b = m._global_rel_bias(300, torch.bfloat16, "cpu")
    assert torch.equal(b[257], b[256])
    assert not torch.equal(b[255], b[254])


def test_mimo_global_matches_brute_force():
    torch.manual_seed(0)
    H, R, D, L, B, thr = 2, 4, 3, 17, 2, 0.05
    m = ot.TESMMIMO_Optimized(d_model=16, d_state=D, n_heads=H, mimo_rank=2, ent_rank=R, entanglement_window=0,
                              entanglement_threshold=thr, max_seq_len=64).eval()
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, L, H, R, generator=g)
    k = torch.randn(B, L, H, R, generator=g)
    S = torch.randn(B, L, H, D, generator=g)
    with torch.no_grad():
        ent, chg = m._global_ent_mimo(q, k, S)
        bias = m._global_rel_bias(L, torch.float32, "cpu").double().numpy()
    qn, kn, sn = q.double().numpy().reshape(B, L, H * R), k.double().numpy().reshape(B, L, H * R), \
        S.double().numpy().reshape(B, L, H * D)
    want = np.zeros((B, L, H * D))
    close = np.zeros((B, L), dtype=bool)
    for b in range(B):
        for i in range(L):
            tern = []
            for j in range(i + 1):
                s = float(qn[b, i] @ kn[b, j]) / math.sqrt(H * R) + bias[i, j]
                close[b, i] |= abs(abs(s) - thr) < 1e-5
                tern.append(1.0 if s > thr else (-1.0 if s < -thr else 0.0))
            n = max(sum(abs(t) for t in tern), 1.0)
            want[b, i] = sum((t / n) * sn[b, j] for j, t in enumerate(tern))
    got = ent.double().numpy().reshape(B, L, H * D)
    ok = ~close
    assert ok.sum() > 0.9 * ok.size
    np.testing.assert_allclose(got[ok], want[ok], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(chg.double().numpy(), (ent - S).double().numpy(), rtol=0, atol=0)
