"""GPU checks of the register-mix entanglement kernel (ent_reg_kernel), the fused SISO entanglement for
the shapes whose state halo fits neither older fused kernel's LDS: float32 rows of 384-512 channels (the
base() preset's d_state 384 / window 32 and the tiny() preset's d_state 384 / rank 96 in float32), which
otherwise take the scores + mix kernels and two activation quantizations.

The kernel forms the window entanglement and the per-token int8 codes of tanh(E) and C (tesm.py:921-952,
1231-1232, 206-209) with one thread per (channel, 8 positions): window sums from registers, weights
broadcast from LDS.  It performs the same float operations in the same order as the older kernels (and,
for bf16, fused multiply-adds whose products are exact), so it is checked bit for bit against them
(TESM_HIP_NO_ENT_REG=1: the scores + mix kernels and the activation quantization), on the isolated op and
inside whole layers.
"""
import pytest
import torch

from hip_helpers import DEV, need_gpu
from tesm_amd import TESM_SISO, hip_ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _case(B, L, R, D, W, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, R, generator=g).to(dtype).to(DEV)
    k = torch.randn(B, L, R, generator=g).to(dtype).to(DEV)
    S = torch.randn(B, L, D, generator=g).to(dtype).to(DEV)
    bias = (torch.randn(W, generator=g) * 0.3).to(DEV)
    cq = torch.randn(B, L, R, generator=g).to(dtype).to(DEV)
    return q, k, S, bias, cq


def _fused2_fits(R, D, weff):
    """The 32-threads-per-position kernel's limits as the library states them (the library's first choice)."""
    rows, half, nsl = 16 + weff - 1, R // 2, D // 8
    lds = (rows * (R + 4) * 4 + 16 * (R + 4) * 4 + 16 * weff * 4 + 15) // 16 * 16 + rows * nsl * 32
    return (D % 16 == 0 and D <= 512 and rows * nsl <= 2048 and rows * half <= 2048 and 16 * half <= 1024
            and weff <= 64 and lds <= 65536)


def _fused16_fits(R, D, weff, dtype):
    """The 16-threads-per-position kernel's limits (the library's second choice): D up to 512, its staged
    keys, queries, weights and state rows within 64 KB."""
    es = 2 if dtype == torch.bfloat16 else 4
    rows, krs, dp = 16 + weff - 1, R + 4, (D + 15) // 16 * 16
    sx = (rows * krs * 4 + 16 * krs * 4 + 16 * weff * 4 + 15) // 16 * 16
    return D <= 512 and (sx + rows * dp * es + 15) // 16 * 16 <= 65536


def _reg_fits(L, D, R, W, dtype):
    """The register-mix kernel's range: D a multiple of 64 up to 512, an effective window of at most 32, LDS
    (staged keys / queries and weights of 16 positions, or the tanh(E) / C staging) within 64 KB."""
    weff = min(W, L)
    wm = 16 if weff <= 16 else 32
    es = 2 if dtype == torch.bfloat16 else 4
    al = lambda v: (v + 15) // 16 * 16  # noqa: E731
    qr = al((16 + weff - 1) * (R + 4) * 4)
    wn = al(qr + 16 * (R + 4) * 4)
    end_wn = wn + 16 * wm * 4
    e1, e2 = 16 * D * es, 32 * D * es
    total = max(end_wn, e2 if (e2 <= end_wn or e2 <= 65536) else e1)
    return D % 64 == 0 and D <= 512 and weff <= 32 and total <= 65536


# (B, L, R, D, W, cross): the base() preset's d_state 384 / window 32, the tiny() preset's d_state 384 /
# rank 96, d_state 512 at window 32, ragged position blocks, windows between 17 and 32, shorter sequences
# than the window, a wide rank on a small block (staging beyond the first round)
SHAPES = [(2, 130, 64, 384, 32, False), (1, 77, 96, 384, 16, True), (1, 96, 32, 512, 32, True),
          (2, 300, 64, 384, 24, False), (1, 12, 64, 384, 32, False), (2, 1, 8, 512, 32, False),
          (1, 40, 128, 448, 17, True), (4, 2048, 64, 384, 32, False)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}xL{}_R{}_D{}_W{}{}".format(*s[:5], "_cross" if s[5] else ""))
def test_ent_reg_matches_older_kernels(shape, dtype, monkeypatch):
    """Codes, scales, row sums, the ternary map and the float tanh(E) / C of the isolated op equal the older
    kernels' bit for bit (the scores + mix kernels and the activation quantization where nothing else fits)."""
    B, L, R, D, W, cross = shape
    q, k, S, bias, cq = _case(B, L, R, D, W, dtype, seed=B * 1000 + L + D + W)
    qa = cq if cross else None
    rope = hip_ops.rope_table(L, R, dtype, DEV)
    weff = min(W, L)
    with hip_ops.launch_log() as log:
        got = hip_ops.local_ent_quant(q, k, rope, S, bias, W, 0.08, 0.2, q_add=qa, want_floats=True, want_tern=True)
        torch.cuda.synchronize()
    expect_reg = _reg_fits(L, D, R, W, dtype) and not _fused2_fits(R, D, weff) and not _fused16_fits(R, D, weff, dtype)
    assert any(k_.startswith("ent_reg_kernel<") for k_ in log.kernels) == expect_reg, log.kernels
    monkeypatch.setenv("TESM_HIP_NO_ENT_REG", "1")
    with hip_ops.launch_log() as log1:
        try:
            ref = hip_ops.local_ent_quant(q, k, rope, S, bias, W, 0.08, 0.2, q_add=qa, want_floats=True,
                                          want_tern=True)
        except RuntimeError as err:  # no older fused form fits: compare with the unfused kernels
            assert "fused quantization needs" in str(err)
            monkeypatch.setenv("TESM_HIP_ENT_UNFUSED", "1")
            fl = hip_ops.local_ent(q, k, rope, S, bias[-weff:], weff, 0.08, 0.2, q_add=qa, outputs=("e_tanh", "c"),
                                   want_tern=True)
            ref = {"tern": fl["tern"][:, :, 0, :], "e_tanh": fl["e_tanh"], "c_float": fl["c"],
                   "te": hip_ops.quant_act(fl["e_tanh"].reshape(B * L, D)),
                   "c": hip_ops.quant_act(fl["c"].reshape(B * L, D))}
        torch.cuda.synchronize()
    assert not any(k_.startswith("ent_reg_kernel<") for k_ in log1.kernels), log1.kernels
    assert torch.equal(got["tern"], ref["tern"])
    assert torch.equal(got["e_tanh"], ref["e_tanh"]) and torch.equal(got["c_float"], ref["c_float"])
    for name in ("te", "c"):
        for a, b in zip(got[name], ref[name]):
            assert torch.equal(a, b), name


# (B, L, d_model, d_state, ent_rank, window, dtype): the base() preset's own d_state 384 / window 32 and the
# tiny() preset's layer (d_state 384, rank 96), d_state 512 / window 32 with a ragged length and a
# cross-layer state, all float32
LAYERS = [(2, 1100, 768, 384, 64, 32, torch.float32), (2, 256, 768, 384, 96, 16, torch.float32),
          (2, 333, 128, 512, 16, 32, torch.float32)]


@pytest.mark.parametrize("shape", LAYERS, ids=lambda s: "B{}xL{}_D{}_R{}_W{}_{}".format(*s[:2], *s[3:6], str(s[6])[6:]))
def test_layer_ent_reg_matches_older_kernels(shape, monkeypatch):
    """The whole SISO prefill with the register-mix kernel gives the same output and final state bits as
    with the unfused kernels (the scan is shared, the entanglement codes are identical)."""
    B, L, dm, D, R, W, dtype = shape
    torch.manual_seed(B + L + D)
    m = TESM_SISO(d_model=dm, d_state=D, ent_rank=R, entanglement_window=W, entanglement_threshold=0.08,
                  entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=L).to(DEV).to(dtype).eval()
    u = torch.randn(B, L, dm, generator=torch.Generator().manual_seed(L)).to(dtype).to(DEV)
    cs = torch.randn(B, L, D, generator=torch.Generator().manual_seed(7)).to(dtype).to(DEV) if L == 333 else None
    with torch.no_grad():
        with hip_ops.launch_log() as log:
            y, f = m(u, cross_layer_state=cs)
        monkeypatch.setenv("TESM_HIP_NO_ENT_REG", "1")
        with hip_ops.launch_log() as log1:
            y1, f1 = m(u, cross_layer_state=cs)
    torch.cuda.synchronize()
    assert any(k_.startswith("ent_reg_kernel<") for k_ in log.kernels), log.kernels
    assert not any(k_.startswith("ent_reg_kernel<") for k_ in log1.kernels), log1.kernels
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y, y1) and torch.equal(f, f1)
