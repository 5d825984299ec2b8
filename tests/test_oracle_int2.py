"""CPU tests of the INT2 export format: the oracle restatement pinned against the reference's
known answers and closed forms, and the host side of the hip loader (validation, layout,
save/load) on CPU modules."""
import os

import numpy as np
import pytest
import torch

from oracle import int2_export as oe
from oracle import int_ref
from oracle import tesm_torch as ot
from tesm_amd import BitLinear, hip_ops
from tesm_amd import int2 as hi


def test_reference_known_answer():
    """[-1, 0, +1, 0] -> 0x64 (int2_quantization.py:12-13); mean|w| = 0.5 gives scale 2."""
    packed, scale = oe.pack_int2_to_uint8(torch.tensor([[-1.0, 0.0, 1.0, 0.0]]))
    assert float(scale) == 2.0
    assert packed.dtype == torch.uint8 and packed.numpy().tolist() == [[0x64]]


def test_hand_computed_scale_codes_and_padding():
    # mean|w| = 1.6/5 = 0.32 -> scale 3.125; w * scale = [1.5625, -1.5625, 0.3125, 0, 1.5625]
    # -> codes [1, -1, 0, 0, 1] -> fields [2, 0, 1, 1 | 2, pad 1, 1, 1] -> bytes 0x52, 0x56
    w = torch.tensor([[0.5, -0.5, 0.1, 0.0, 0.5]])
    packed, scale = oe.pack_int2_to_uint8(w)
    assert float(scale) == pytest.approx(3.125, rel=1e-7)
    assert packed.numpy().tolist() == [[0x52, 0x56]]
    deq = oe.unpack_uint8_to_int2(packed, float(scale))
    np.testing.assert_array_equal(deq.numpy()[:, :5] * 3.125, [[1, -1, 0, 0, 1]])
    assert deq.shape == (1, 8) and float(deq[0, 5:].abs().sum()) == 0.0


def test_reference_shape_assertion():
    """16 x 64 weight -> 16 x 16 uint8 (tests/test_torch_only.py:398-403)."""
    packed, _ = oe.pack_int2_to_uint8(torch.randn(16, 64))
    assert packed.shape == (16, 16) and packed.dtype == torch.uint8


def test_all_zero_weight_uses_export_clamp():
    """The export clamps mean|w| at 1e-8 (int2_quantization.py:32), not at BitLinear's 1e-5."""
    packed, scale = oe.pack_int2_to_uint8(torch.zeros(3, 9))
    assert float(scale) == pytest.approx(1e8, rel=1e-7)
    assert np.all(packed.numpy()[:, :2] == 0x55) and np.all(packed.numpy()[:, 2] == 0x55)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_export_dequantizes_to_bitlinear_weight(dtype):
    """unpack(export) reproduces BitLinear.quantized_weight (tesm.py:211-215) whenever
    mean|w| >= bit_eps: the export and the module quantize alike."""
    torch.manual_seed(5)
    bl = ot.BitLinear(70, 12).to(dtype)
    packed, scale = oe.pack_int2_to_uint8(bl.weight.data)
    assert packed.shape == (12, 18)
    codes = int_ref.unpack_i2(packed.numpy(), 70)
    with torch.no_grad():
        qw = bl.quantized_weight()
        s = bl.weight_scale()
    assert float(s) == float(scale)
    np.testing.assert_array_equal(codes, (qw * s).round().float().numpy())
    deq = (torch.from_numpy(codes).to(dtype) / scale)
    assert torch.equal(deq, qw)


def test_export_model_entries():
    torch.manual_seed(0)
    m = ot.TESM_SISO(d_model=64, d_state=16, ent_rank=8, entanglement_window=4, max_seq_len=64)
    ex = oe.export_model_to_int2(m)
    names = {n for n, mod in m.named_modules() if isinstance(mod, ot.BitLinear)}
    assert set(ex) == names and len(names) >= 4
    for name, e in ex.items():
        mod = dict(m.named_modules())[name]
        assert e["packed_weight"].shape == (mod.out_features, (mod.in_features + 3) // 4)
        assert e["in_features"] == mod.in_features and e["out_features"] == mod.out_features
        assert e["weight_scale"].dim() == 0


# ---------------------------------------------------------------------------
# host side of tesm_amd.int2 on CPU modules (no kernels run)
# ---------------------------------------------------------------------------
def _entry(N, K, seed=0):
    w = torch.randn(N, K, generator=torch.Generator().manual_seed(seed))
    packed, scale = oe.pack_int2_to_uint8(w)
    return {"packed_weight": packed, "weight_scale": scale, "bias": None, "in_features": K, "out_features": N}


def test_load_lays_out_codes_for_the_products():
    e = _entry(6, 70)
    bl = BitLinear(70, 6)
    bl.load_int2(**e)
    assert bl.is_int2
    pw = bl._int2_cache(torch.float32, torch.device("cpu"))
    kb = 18
    assert pw.packed.shape == (6, hip_ops.kpad(70) // 4)
    assert np.array_equal(pw.packed.numpy()[:, :kb], e["packed_weight"].numpy())
    assert np.all(pw.packed.numpy()[:, kb:] == 0x55)
    s = float(e["weight_scale"])
    assert float(pw.s_w[0]) == s
    assert float(pw.c_w[0]) == float(torch.tensor(1.0) / torch.tensor(s))


def test_load_rounds_scale_to_module_dtype():
    e = _entry(4, 16, seed=2)
    bl = BitLinear(16, 4).to(torch.bfloat16)
    bl.load_int2(**e)
    pw = bl._int2_cache(torch.bfloat16, torch.device("cpu"))
    s_bf = torch.tensor(float(e["weight_scale"])).to(torch.bfloat16)
    assert float(pw.s_w[0]) == float(s_bf)
    assert float(pw.c_w[0]) == float(torch.ones((), dtype=torch.bfloat16) / s_bf)


def test_load_normalizes_pad_fields():
    e = _entry(3, 5, seed=3)
    p = e["packed_weight"].clone()
    p[:, 1] = (p[:, 1] & 0x03) | 0x00  # pad fields set to code 0 instead of 1
    bl = BitLinear(5, 3)
    bl.load_int2(p, e["weight_scale"])
    assert np.array_equal(bl.int2_packed.numpy(), e["packed_weight"].numpy())


def test_load_rejects_bad_entries():
    e = _entry(4, 8)
    bl = BitLinear(8, 4)
    with pytest.raises(ValueError, match="layer is 8 -> 4"):
        bl.load_int2(**dict(e, in_features=12))
    with pytest.raises(ValueError, match="uint8 of shape"):
        bl.load_int2(e["packed_weight"][:, :1], e["weight_scale"])
    with pytest.raises(ValueError, match="uint8 of shape"):
        bl.load_int2(e["packed_weight"].to(torch.int16), e["weight_scale"])
    bad = e["packed_weight"].clone()
    bad[1, 0] |= 0x0C  # field 1 = 3
    with pytest.raises(ValueError, match="equal to 3"):
        bl.load_int2(bad, e["weight_scale"])
    for s in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="positive finite"):
            bl.load_int2(e["packed_weight"], torch.tensor(s))
    with pytest.raises(ValueError, match="one value"):
        bl.load_int2(e["packed_weight"], torch.ones(2))
    with pytest.raises(ValueError, match="bias must have"):
        bl.load_int2(e["packed_weight"], e["weight_scale"], bias=torch.zeros(3))
    assert not bl.is_int2


def test_load_bias_and_release_and_clear():
    e = _entry(4, 8)
    bl = BitLinear(8, 4, bias=True)
    key0 = bl.cache_key()
    bl.load_int2(**e)  # bias None in the entry removes the layer's bias, as the module swap does
    assert bl.bias is None and bl.cache_key() != key0
    b = torch.arange(4, dtype=torch.float32)
    bl.load_int2(e["packed_weight"], e["weight_scale"], bias=b, keep_float_weight=False)
    assert torch.equal(bl.bias.data, b) and bl.weight.numel() == 0 and bl.weight.dtype == torch.float32
    with pytest.raises(RuntimeError, match="released"):
        bl.clear_int2()
    bl2 = BitLinear(8, 4)
    bl2.load_int2(**e)
    bl2.clear_int2()
    assert not bl2.is_int2


def test_loader_skips_unknown_names_and_round_trips_through_file(tmp_path):
    torch.manual_seed(1)
    ref = ot.TESM_SISO(d_model=64, d_state=16, ent_rank=8, entanglement_window=4, max_seq_len=64)
    ex = oe.export_model_to_int2(ref)
    ex["no_such_layer"] = _entry(2, 4)
    path = os.path.join(tmp_path, "int2.pt")
    torch.save(ex, path)
    torch.manual_seed(2)
    from tesm_amd import TESM_SISO
    m = TESM_SISO(d_model=64, d_state=16, ent_rank=8, entanglement_window=4, max_seq_len=64)
    loaded = hi.load_int2_model(m, path)
    assert set(loaded) == set(ex) - {"no_such_layer"}
    for name in loaded:
        mod = dict(m.named_modules())[name]
        assert np.array_equal(mod.int2_packed.numpy(), ex[name]["packed_weight"].numpy())
        assert mod.int2_scale == float(ex[name]["weight_scale"])
    # an INT2-backed model exports the entries it was loaded from
    back = hi.export_model_to_int2(m)
    for name in loaded:
        assert torch.equal(back[name]["packed_weight"], ex[name]["packed_weight"])
        assert float(back[name]["weight_scale"]) == float(ex[name]["weight_scale"])
