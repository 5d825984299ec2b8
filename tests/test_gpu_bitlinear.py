"""GPU parity of the BitLinear pieces (C-ABI through tesm_amd.hip_ops) against the oracle.

Bar: int8 activation codes, activation scales, packed INT2 bytes and int32
accumulators bit-exact; float outputs within 1e-3 (fp32) / 2e-2 (bf16) normwise.
"""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from hip_helpers import DEV, TOL, bf16_bits, need_gpu, normwise, to_np, unpermute_layout1
from oracle import int_ref
from oracle import tesm_torch as ot
from tesm_amd import BitLinear, hip_ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _oracle_codes(x: torch.Tensor):
    if x.dtype == torch.bfloat16:
        return int_ref.quant_act(bf16_bits(x), bf16_bits=True)
    return int_ref.quant_act(x.numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,K", [(1, 64), (3, 61), (5, 130), (17, 768), (2, 4096), (64, 256),
                                 (2048, 384), (2048, 768), (2050, 1024)])  # last three: 16 lanes per row
def test_quant_act_bit_exact(dtype, M, K):
    g = torch.Generator().manual_seed(M * 1000 + K)
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    if M > 2:
        x[1] = 0                                  # all-zero row -> eps clamp, zero codes
        x[2, : K // 2] = 0.5 * x[2, : K // 2].sign()  # repeated magnitudes
    q_ref, s_ref = _oracle_codes(x)
    xd = x.to(DEV)
    for layout in (0, 1):
        q, s, rs = hip_ops.quant_act(xd, layout=layout)
        torch.cuda.synchronize()
        qn = q.cpu().numpy()
        codes = qn[:, :K] if layout == 0 else unpermute_layout1(qn, K)
        assert np.array_equal(codes, q_ref), f"layout {layout}"
        if layout == 0:
            assert np.all(qn[:, K:] == 0)
        assert np.array_equal(s.cpu().numpy(), s_ref)
        assert np.array_equal(rs.cpu().numpy(), q_ref.astype(np.int64).sum(1))
    # codes past K (padding up to kpad) must be zero
    q, _, _ = hip_ops.quant_act(xd, layout=1)
    assert np.all(unpermute_layout1(q.cpu().numpy(), q.shape[1])[:, K:] == 0)


def test_quant_act_ties_round_half_even():
    # amax 127 -> scale exactly 1: codes are rne(x); .5 ties go to even
    x = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.0, 3.49999]], dtype=torch.float32)
    q, s, _ = hip_ops.quant_act(x.to(DEV), layout=0)
    q_ref, s_ref = _oracle_codes(x)
    assert np.array_equal(q.cpu().numpy()[:, :10], q_ref)
    assert q_ref[0, 1] == 0 and q_ref[0, 2] == 2 and q_ref[0, 3] == 2 and q_ref[0, 7] == 126


def test_quant_act_strided_rows():
    x = torch.randn(6, 300)
    view = x[:, 20:148]                               # row stride 300, width 128
    q_ref, s_ref = _oracle_codes(view.contiguous())
    q, s, _ = hip_ops.quant_act(x.to(DEV)[:, 20:148], layout=0)
    assert np.array_equal(q.cpu().numpy()[:, :128], q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_absmean_scale(dtype):
    w = (torch.randn(300, 77, generator=torch.Generator().manual_seed(3)) * 0.02).to(dtype)
    s_ref = (1.0 / w.abs().mean().clamp_min(1e-5))
    s_w, c_w = hip_ops.absmean_scale(w.to(DEV))
    s = s_w.cpu()[0]
    # the fp64 device reduction may differ from torch's CPU order by one ulp of the mean
    ulp = float(torch.finfo(dtype).eps) * abs(float(s_ref))
    assert abs(float(s) - float(s_ref)) <= ulp
    c_ref = (torch.ones((), dtype=dtype) / s.to(dtype)).float()
    assert float(c_w.cpu()[0]) == float(c_ref)
    # all-zero weights hit the eps clamp
    s0, _ = hip_ops.absmean_scale(torch.zeros(8, 8, dtype=dtype, device=DEV))
    assert float(s0.cpu()[0]) == float((1.0 / torch.tensor(1e-5, dtype=dtype)).float())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,K", [(40, 64), (24, 130), (7, 61), (96, 768)])
def test_pack_bit_exact(dtype, N, K):
    w = (torch.randn(N, K, generator=torch.Generator().manual_seed(N + K)) * 0.02).to(dtype)
    s_w = (1.0 / w.float().abs().mean()).to(dtype).float().reshape(1)  # any scale: codes are checked given s_w
    if dtype == torch.bfloat16:
        codes = int_ref.weight_codes(bf16_bits(w), float(s_w), bf16_bits=True)
    else:
        codes = int_ref.weight_codes(w.numpy(), float(s_w))
    ref = int_ref.pack_i2(codes)
    canon = hip_ops.pack_weight(w.to(DEV), s_w.to(DEV), ldp=(K + 3) // 4)
    assert np.array_equal(canon.cpu().numpy(), ref)
    padded = hip_ops.pack_weight(w.to(DEV), s_w.to(DEV)).cpu().numpy()
    kb = (K + 3) // 4
    assert np.array_equal(padded[:, :kb], ref) and np.all(padded[:, kb:] == 0x55)
    back = hip_ops.unpack_weight(canon, K).cpu().numpy()
    assert np.array_equal(back, codes)


def test_pack_known_answer():
    """[-1, 0, +1, 0] -> 0x64 (tesm_ssm/utils/int2_quantization.py:12-13)."""
    w = torch.tensor([[-1.0, 0.0, 1.0, 0.0]], device=DEV)
    p = hip_ops.pack_weight(w, torch.ones(1, device=DEV), ldp=1)
    assert p.cpu().numpy()[0, 0] == 0x64
    g = load_golden("pack_kat")
    codes = torch.from_numpy(g["codes"].astype(np.float32)).to(DEV)
    p = hip_ops.pack_weight(codes, torch.ones(1, device=DEV), ldp=g["packed"].shape[1])
    assert np.array_equal(p.cpu().numpy(), g["packed"])


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 16, 32, 33, 64, 65, 200])
@pytest.mark.parametrize("K,N", [(64, 40), (130, 24), (768, 200), (4096, 64), (256, 300)])
def test_accumulators_bit_exact(M, K, N):
    """int32 accumulators of the GEMV (M <= 4) and MFMA (M > 4) paths vs the exact integer product."""
    g = torch.Generator().manual_seed(M * 7 + K * 3 + N)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g)
    s_w = (1.0 / w.abs().mean()).reshape(1)
    q_ref, s_ref = int_ref.quant_act(x.numpy())
    wc = int_ref.weight_codes(w.numpy(), float(s_w))
    acc_ref = int_ref.bitlinear_acc(q_ref, wc)
    q, s, rs = hip_ops.quant_act(x.to(DEV))
    packed = hip_ops.pack_weight(w.to(DEV), s_w.to(DEV))
    c_w = (1.0 / s_w).to(DEV)
    out, acc = hip_ops.bitlinear(q, s, rs, packed, c_w, N, K, torch.float32, acc_dump=True)
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    y_ref = acc_ref.astype(np.float64) / s_ref.astype(np.float64)[:, None] * float(c_w.cpu()[0])
    assert normwise(out.cpu().numpy(), y_ref) < 1e-6


@pytest.mark.parametrize("name", ["bl_f32_small", "bl_f32_padk", "bl_f32_gemv", "bl_bf16_small", "bl_bf16_gemv"])
def test_bitlinear_module_vs_reference_fixture(name):
    """The hip BitLinear module on the reference's own inputs: codes/bytes exact, output within tolerance."""
    g, meta = load_golden(name), golden_meta(name)
    dt = torch.bfloat16 if meta["dtype"] == "torch.bfloat16" else torch.float32
    M, K, N = meta["M"], meta["K"], meta["N"]
    bl = BitLinear(K, N).to(DEV)
    with torch.no_grad():
        bl.weight.copy_(torch.from_numpy(g["weight"]))
    bl = bl.to(dt).eval()
    x = torch.from_numpy(g["x"]).to(dt).to(DEV)
    with torch.no_grad():
        y = bl(x)
        pw = bl.packed_weight()
        q, s, _ = hip_ops.quant_act(x, layout=0)
    assert np.array_equal(q.cpu().numpy()[:, :K], g["x_codes"])
    assert np.array_equal(s.cpu().numpy(), g["s_x"])
    # packed bytes given the reference's scale (the device mean may differ in the last bit)
    canon = hip_ops.pack_weight(bl.weight.detach(), torch.from_numpy(g["s_w"]).to(DEV), ldp=(K + 3) // 4)
    assert np.array_equal(canon.cpu().numpy(), g["packed"])
    assert pw.packed.shape == (N, hip_ops.kpad(K) // 4)
    assert normwise(to_np(y), g["y"]) <= TOL[dt]


def test_bitlinear_module_shapes_and_cache():
    bl = BitLinear(256, 96).to(DEV).eval()
    x = torch.randn(2, 7, 256, device=DEV)
    with torch.no_grad():
        y1 = bl(x)
        p1 = bl.packed_weight()
        y2 = bl(x)
        assert bl.packed_weight() is p1            # cached while the weight version is unchanged
        bl.weight.mul_(-1.0)
        y3 = bl(x)
    assert y1.shape == (2, 7, 96)
    assert torch.equal(y1, y2)
    assert torch.allclose(y3, -y1)
    ref = ot.BitLinear(256, 96)
    with torch.no_grad():
        ref.weight.copy_(bl.weight.cpu())
        yr = ref.eval()(x.cpu())
    assert normwise(to_np(y3), yr.numpy()) <= 1e-3


def test_bitlinear_strict_errors():
    bl = BitLinear(64, 8).to(DEV)
    x = torch.randn(1, 64, device=DEV)
    with pytest.raises(RuntimeError, match="kernel_backend"):
        bl.train()(x)
    with pytest.raises(RuntimeError, match="kernel_backend"):
        bl.eval()(x)  # grad enabled
    with torch.no_grad(), pytest.raises(RuntimeError, match="kernel_backend"):
        BitLinear(64, 8, kernel_backend="torch").to(DEV).eval()(x)


@pytest.mark.parametrize("M,K,N,ragged", [(16384, 2048, 4096, False), (16388, 2100, 4096, True), (2048, 768, 2432, False),
                                          (4096, 4096, 256, False), (4096, 2048, 1024, False),
                                          (32, 2048, 34816, False), (20, 1000, 17000, True), (5, 4096, 16400, False),
                                          (8192, 768, 2432, False), (8000, 700, 2400, True)])
def test_accumulators_bit_exact_large(M, K, N, ragged):
    """int32 accumulators of the large-tile GEMMs (direct-to-LDS main loop for K >= 2048 when N fills
    256-wide tiles; register-staged otherwise; 32-row tiles for decode-size batches over wide weights;
    128x256 then 128x128 tiles in one launch for the in_proj shape)
    vs the exact product: integer-valued float32 matrices multiply exactly on the device while |sums| <
    2^24 (here <= 127 * K)."""
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(DEV)
    w = torch.randn(N, K, generator=g).to(DEV)
    s_w = (1.0 / w.abs().mean()).reshape(1)
    q, s, rs = hip_ops.quant_act(x)
    packed = hip_ops.pack_weight(w, s_w)
    c_w = 1.0 / s_w
    out, acc = hip_ops.bitlinear(q, s, rs, packed, c_w, N, K, torch.float32, acc_dump=True)
    codes = hip_ops.unpack_weight(packed, K).to(torch.float32)                    # (N, K) in {-1, 0, 1}
    from hip_helpers import unpermute_layout1
    xq = torch.from_numpy(unpermute_layout1(q.cpu().numpy()[:, : hip_ops.kpad(K)], K)).to(DEV).to(torch.float32)
    acc_ref = (xq @ codes.t().contiguous()).to(torch.int64)
    assert torch.equal(acc.to(torch.int64), acc_ref)
    y_ref = (acc_ref.to(torch.float64) / s.to(torch.float64)[:, None]) * float(c_w.cpu()[0])
    assert normwise(out.cpu().numpy(), y_ref.cpu().numpy()) < 1e-6
    # the plain (no dump) epilogue path writes the same values
    out2 = hip_ops.bitlinear(q, s, rs, packed, c_w, N, K, torch.float32)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("M,K,N", [(8192, 768, 2432), (32, 2048, 34816), (20, 1000, 3000), (2048, 4096, 4096),
                                   (300, 768, 200)])
def test_per_row_scale_and_bias_epilogue(M, K, N):
    """Per-output-column weight scales (the grouped feed-forward's layout) and a bias through every
    product family (split in_proj tiles, wide decode tiles, split-K, large tiles, small tiles): the
    float32 output equals ((acc - rowsum) * (1 / s_x)) * c_w[n] + bias[n], each op one float32
    rounding, computed from the kernel's own int32 accumulators (whose exactness the tests above pin)."""
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g).to(DEV)
    w = torch.randn(N, K, generator=g).to(DEV)
    s_w = (1.0 / w.abs().mean(dim=1)).to(torch.float32)                 # one scale per output row of w
    q, s, rs = hip_ops.quant_act(x)
    packed = hip_ops.pack_weight(w, s_w, per_row=True)
    c_w = (1.0 / s_w).contiguous()
    bias = torch.randn(N, generator=g).to(DEV)
    out, acc = hip_ops.bitlinear(q, s, rs, packed, c_w, N, K, torch.float32, bias=bias, c_w_per_row=True,
                                 acc_dump=True)
    inv = 1.0 / s                                                       # float32, as the kernels form it
    ref = (acc.to(torch.float32) * inv[:, None]) * c_w[None, :] + bias[None, :]
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    out2 = hip_ops.bitlinear(q, s, rs, packed, c_w, N, K, torch.float32, bias=bias, c_w_per_row=True)
    assert torch.equal(out, out2)
