"""GPU parity of the INT2 export loader (tesm_ssm/utils/int2_quantization.py:196-279).

Bar: exported bytes bit-exact against the oracle's restatement of the export; a
model loaded from an export computes bit-identically to the BitLinear model it was
exported from (same codes, same scale, same kernels); a model loaded from the
oracle's export of a float model matches that float model's oracle forward within
the layer tests' tolerance.
"""
import numpy as np
import pytest
import torch

from flips import Flips, Taps, assert_rows, install, uninstall
from hip_helpers import DEV, TOL, bf16_bits, need_gpu, normwise, to_np
from oracle import int2_export as oe
from oracle import int_ref
from oracle import tesm_torch as ot
from tesm_amd import BitLinear, TESM_SISO, TESMMIMO_Optimized
from tesm_amd import int2 as hi

pytestmark = pytest.mark.gpu

SISO_CFG = dict(d_model=128, d_state=64, ent_rank=16, entanglement_window=16, entanglement_threshold=0.08,
                entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=512)
MIMO_CFG = dict(d_model=128, d_state=32, n_heads=4, mimo_rank=3, ent_rank=16, entanglement_window=16,
                entanglement_threshold=0.05, entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=128)


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _scramble(model):
    """Overwrite every BitLinear float weight and bias, so that only a loaded export can reproduce
    the original outputs."""
    g = torch.Generator().manual_seed(4321)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, BitLinear):
                mod.weight.copy_(torch.randn(mod.weight.shape, generator=g).to(mod.weight.dtype))
                if mod.bias is not None:
                    mod.bias.copy_(torch.randn(mod.bias.shape, generator=g).to(mod.bias.dtype))
    return model


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,K", [(12, 70), (96, 768), (7, 4), (33, 130)])
def test_export_bytes_match_oracle(dtype, N, K):
    torch.manual_seed(N * 31 + K)
    ref = ot.BitLinear(K, N).to(dtype)
    bl = BitLinear(K, N).to(dtype)
    with torch.no_grad():
        bl.weight.copy_(ref.weight)
    bl = bl.to(DEV)
    ex = hi.export_model_to_int2(bl)[""]
    exr = oe.export_model_to_int2(ref)[""]
    assert ex["packed_weight"].dtype == torch.uint8 and ex["packed_weight"].shape == (N, (K + 3) // 4)
    assert ex["weight_scale"].dtype == dtype and ex["weight_scale"].dim() == 0
    # the device mean|w| may differ from torch's CPU reduction order by one ulp (fp32), which the
    # rounded reciprocal can turn into two ulp of the scale
    s, sr = float(ex["weight_scale"]), float(exr["weight_scale"])
    assert abs(s - sr) <= 2 * float(torch.finfo(dtype).eps) * abs(sr)
    w = ref.weight.data
    codes = (int_ref.weight_codes(bf16_bits(w), s, bf16_bits=True) if dtype == torch.bfloat16
             else int_ref.weight_codes(w.numpy(), s))
    assert np.array_equal(ex["packed_weight"].numpy(), int_ref.pack_i2(codes))
    if s == sr:
        assert torch.equal(ex["packed_weight"], exr["packed_weight"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,N,M,bias", [(70, 12, 5, True), (768, 200, 64, False), (256, 96, 1, True)])
def test_bitlinear_round_trip_bit_exact(dtype, K, N, M, bias):
    torch.manual_seed(K + N)
    a = BitLinear(K, N, bias=bias).to(DEV).to(dtype).eval()
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(9)).to(dtype).to(DEV)
    with torch.no_grad():
        ya = a(x)
    ex = hi.export_model_to_int2(a)
    b = _scramble(BitLinear(K, N, bias=not bias).to(DEV).to(dtype).eval())
    assert hi.load_int2_weights_to_model(b, ex) == [""]
    with torch.no_grad():
        yb = b(x)
    assert (b.bias is None) == (not bias)
    assert torch.equal(ya, yb)
    # a changed float weight no longer matters to an INT2-backed layer
    with torch.no_grad():
        b.weight.mul_(-1.0)
        assert torch.equal(b(x), ya)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bitlinear_from_oracle_export_matches_float_model(dtype):
    torch.manual_seed(17)
    ref = ot.BitLinear(300, 150, bias=True).to(dtype).eval()
    x = torch.randn(40, 300, generator=torch.Generator().manual_seed(2)).to(dtype)
    with torch.no_grad():
        yr = ref(x)
    m = BitLinear(300, 150).to(DEV).to(dtype).eval()
    hi.load_int2_weights_to_model(m, oe.export_model_to_int2(ref), keep_float_weights=False)
    assert m.weight.numel() == 0
    with torch.no_grad():
        y = m(x.to(DEV))
    assert normwise(to_np(y), to_np(yr)) <= (1e-5 if dtype == torch.float32 else TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("window", [16, 0])
def test_siso_round_trip_prefill_and_decode_bit_exact(dtype, window):
    cfg = dict(SISO_CFG, entanglement_window=window)
    torch.manual_seed(123)
    a = TESM_SISO(**cfg).to(DEV).to(dtype).eval()
    torch.manual_seed(123)
    b = TESM_SISO(**cfg).to(DEV).to(dtype).eval()
    u = torch.randn(2, 40, 128, generator=torch.Generator().manual_seed(7)).to(dtype).to(DEV)

    def run(m):
        cache = m.allocate_inference_cache(2, 64)
        ip = {"state_cache": cache}
        with torch.no_grad():
            y, f = m(u[:, :32], inference_params=ip)
            outs = [y.clone(), f.clone()]
            for t in range(32, 40 if window else 32):  # hip decode covers windowed layers
                ys, st = m(u[:, t:t + 1], inference_params=ip)
                outs += [ys.clone(), st.clone()]
        return outs

    ra = run(a)
    rb0 = run(b)  # builds b's decode plan from its own float weights first
    assert all(torch.equal(p, q) for p, q in zip(ra, rb0))
    _scramble(b)
    hi.load_int2_weights_to_model(b, hi.export_model_to_int2(a))
    rb = run(b)
    for i, (p, q) in enumerate(zip(ra, rb)):
        assert torch.equal(p, q), i


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_siso_from_oracle_export_matches_float_model(dtype):
    torch.manual_seed(123)
    ref = ot.TESM_SISO(**SISO_CFG).eval().to(dtype)
    torch.manual_seed(123)
    m = _scramble(TESM_SISO(**SISO_CFG).eval()).to(DEV).to(dtype)
    hi.load_int2_weights_to_model(m, oe.export_model_to_int2(ref), keep_float_weights=False)
    u = torch.randn(2, 300, 128, generator=torch.Generator().manual_seed(7)).to(dtype)
    flips = Flips(dtype)
    D, W = SISO_CFG["d_state"], SISO_CFG["entanglement_window"]
    with torch.no_grad():
        with Taps(600, D, 128, DEV, (2, 300, min(W, 300)), d_state=D, dtype=dtype) as tp:
            y, f = m(u.to(DEV))
        install(ref, flips, tp, "local", states=m._last_cross_layer_state)
        yr, fr = ref(u)
        uninstall(ref)
    assert_rows(to_np(y), to_np(yr), dtype, f"INT2-loaded layer ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
    else:
        assert normwise(f.cpu().numpy(), fr.numpy()) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mimo_round_trip_bit_exact(dtype):
    torch.manual_seed(55)
    a = TESMMIMO_Optimized(**MIMO_CFG).to(DEV).to(dtype).eval()
    torch.manual_seed(55)
    b = _scramble(TESMMIMO_Optimized(**MIMO_CFG)).to(DEV).to(dtype).eval()
    u = torch.randn(2, 100, 128, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)
    loaded = hi.load_int2_weights_to_model(b, hi.export_model_to_int2(a))
    assert len(loaded) >= 4
    with torch.no_grad():
        ya, fa = a(u)
        yb, fb = b(u)
    assert torch.equal(ya, yb) and torch.equal(fa, fb)
