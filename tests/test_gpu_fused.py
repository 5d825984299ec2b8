"""GPU parity of the fused kernels: entanglement + int8 quantization of tanh(E) and C, and the
row-complete output gate + out_proj input quantization.

Each fused kernel is checked bit-for-bit against the unfused kernels it replaces (same float
sequence), and the output gate against an integer restatement of the reference formula
y = local + sigmoid(gate) * state_proj(tanh E) + ent_proj(C) (tesm.py:1256-1260).
"""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from hip_helpers import DEV, need_gpu, normwise, to_np
from oracle import int_ref
from tesm_amd import hip_ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _case(B, L, R, D, W, dtype, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, L, R, generator=g) * std).to(dtype).to(DEV)
    k = (torch.randn(B, L, R, generator=g) * std).to(dtype).to(DEV)
    S = torch.randn(B, L, D, generator=g).to(dtype).to(DEV)
    bias = (torch.randn(W, generator=g) * 0.3).to(DEV)
    cq = torch.randn(B, L, R, generator=g).to(dtype).to(DEV)
    return q, k, S, bias, cq


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,R,D,W,cross", [(2, 40, 8, 32, 8, False), (1, 300, 64, 256, 16, True),
                                             (3, 17, 16, 48, 32, False), (1, 5, 8, 512, 8, True),
                                             (2, 130, 64, 384, 32, False)])
def test_fused_entanglement_quant_matches_unfused(dtype, B, L, R, D, W, cross, monkeypatch):
    q, k, S, bias, cq = _case(B, L, R, D, W, dtype, seed=B * 100 + L + D)
    qa = cq if cross else None
    rope = hip_ops.rope_table(L, R, dtype, DEV)
    weff = min(W, L)
    monkeypatch.setenv("TESM_HIP_ENT_UNFUSED", "1")  # the float outputs from the scores + mix kernels
    ref = hip_ops.local_ent(q, k, rope, S, bias[-weff:], weff, 0.08, 0.2, q_add=qa,
                            outputs=("e_tanh", "c"), want_tern=True)
    monkeypatch.delenv("TESM_HIP_ENT_UNFUSED")
    fz = hip_ops.local_ent_quant(q, k, rope, S, bias, W, 0.08, 0.2, q_add=qa, want_floats=True, want_tern=True)
    torch.cuda.synchronize()
    assert torch.equal(fz["tern"], ref["tern"][:, :, 0, :])
    assert torch.equal(fz["e_tanh"], ref["e_tanh"]) and torch.equal(fz["c_float"], ref["c"])
    for name, src in (("te", ref["e_tanh"]), ("c", ref["c"])):
        qr, sr, rr = hip_ops.quant_act(src.reshape(B * L, D))
        qf, sf, rf = fz[name]
        assert torch.equal(qf, qr), name
        assert torch.equal(sf, sr) and torch.equal(rf, rr), name


def _fused2_fits(R, D, weff):
    """The 32-threads-per-position kernel's limits as the library states them: 16-channel multiples up to
    512, at most 4 staged key / state items and 2 query items per thread, its LDS within 64 KB."""
    rows, half, nsl = 16 + weff - 1, R // 2, D // 8
    lds = (rows * (R + 4) * 4 + 16 * (R + 4) * 4 + 16 * weff * 4 + 15) // 16 * 16 + rows * nsl * 32
    return (D % 16 == 0 and D <= 512 and rows * nsl <= 2048 and rows * half <= 2048 and 16 * half <= 1024
            and weff <= 64 and lds <= 65536)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,R,D,W,cross", [(2, 40, 8, 32, 8, False), (1, 300, 64, 256, 16, True),
                                             (3, 17, 16, 48, 32, False), (1, 5, 8, 512, 8, True),
                                             (2, 130, 64, 384, 32, False), (8, 512, 48, 256, 16, False)])
def test_fused_entanglement_float_outputs_match_unfused(dtype, B, L, R, D, W, cross, monkeypatch):
    """The float-output entry (window average, E, C, tanh(E); tesm.py:921-952, 1231-1232) on the
    32-threads-per-position kernel equals the scores + mix kernels bit for bit, ternary map included."""
    q, k, S, bias, cq = _case(B, L, R, D, W, dtype, seed=B * 100 + L + D + 7)
    qa = cq if cross else None
    rope = hip_ops.rope_table(L, R, dtype, DEV)
    weff = min(W, L)
    names = ("avg", "e", "c", "e_tanh")
    with hip_ops.launch_log() as log:
        got = hip_ops.local_ent(q, k, rope, S, bias[-weff:], weff, 0.08, 0.2, q_add=qa, outputs=names, want_tern=True)
        torch.cuda.synchronize()
    monkeypatch.setenv("TESM_HIP_ENT_UNFUSED", "1")
    with hip_ops.launch_log() as log1:
        ref = hip_ops.local_ent(q, k, rope, S, bias[-weff:], weff, 0.08, 0.2, q_add=qa, outputs=names, want_tern=True)
        torch.cuda.synchronize()
    fits = _fused2_fits(R, D, weff)
    assert any(k_.startswith("ent_fused2_kernel<") for k_ in log.kernels) == fits, log.kernels
    assert not any(k_.startswith("ent_fused2_kernel<") for k_ in log1.kernels), log1.kernels
    for name in names + ("tern",):
        assert torch.equal(got[name], ref[name]), name


@pytest.mark.parametrize("name", ["siso_f32", "siso_bf16", "siso_f32_widerank"])
def test_fused_entanglement_on_reference_stage_inputs(name):
    """Identity RoPE + the reference's own q, k, states: codes equal the oracle's quantization of
    tanh(E) and C computed from the reference's entanglement output."""
    g, meta = load_golden(name), golden_meta(name)
    dt = torch.bfloat16 if meta["dtype"] == "torch.bfloat16" else torch.float32
    q = torch.from_numpy(g["_compute_entanglement/arg0#0"]).to(dt)
    k = torch.from_numpy(g["_compute_entanglement/arg1#0"]).to(dt)
    S = torch.from_numpy(g["_compute_entanglement/arg2#0"]).to(dt)
    B, L, R = q.shape
    D = S.shape[-1]
    rope = torch.zeros(L, R // 2, 2, device=DEV)
    rope[..., 0] = 1.0
    bias = torch.from_numpy(g["param/local_entanglement_bias"])
    fz = hip_ops.local_ent_quant(q.to(DEV), k.to(DEV), rope, S.to(DEV), bias, meta["W"], meta["thr"], meta["scale"])
    avg = torch.from_numpy(g["_compute_entanglement/out#0"]).to(dt)
    e = S + meta["scale"] * (avg - S)                                   # tesm.py:1231-1232 in dtype
    for nm, x in (("te", torch.tanh(e)), ("c", e - S)):
        x2 = x.reshape(B * L, D)
        if dt == torch.bfloat16:
            from hip_helpers import bf16_bits
            codes, s = int_ref.quant_act(bf16_bits(x2), bf16_bits=True)
        else:
            codes, s = int_ref.quant_act(x2.numpy())
        from hip_helpers import unpermute_layout1
        got = unpermute_layout1(fz[nm][0].cpu().numpy(), D)
        # tanh on the device may differ from torch's CPU tanh in the last bit
        agree = (got == codes).mean()
        exact = nm == "c" and dt == torch.float32   # no transcendental and no bf16 avg rounding
        assert agree >= (1.0 if exact else 0.999), (nm, agree)
        assert np.abs(got.astype(int) - codes.astype(int)).max() <= 1
        np.testing.assert_allclose(fz[nm][1].cpu().numpy(), s, rtol=2 ** -7)


def _codes(x):
    return hip_ops.quant_act(x)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,dm,D", [(37, 64, 32), (300, 768, 256), (16, 96, 64), (129, 1024, 384), (5, 200, 130),
                                    (4096, 1024, 256)])
def test_output_gate_vs_integer_reference(dtype, M, dm, D):
    g = torch.Generator().manual_seed(M + dm + D)
    te_x = torch.tanh(torch.randn(M, D, generator=g)).to(dtype)
    c_x = (torch.randn(M, D, generator=g) * 0.1).to(dtype)
    local = torch.randn(M, dm, generator=g).to(dtype)
    gate = torch.randn(M, dm, generator=g).to(dtype)
    w_sp = torch.randn(dm, D, generator=g) * 0.02
    w_ep = torch.randn(dm, D, generator=g) * 0.02
    te = _codes(te_x.to(DEV))
    cc = _codes(c_x.to(DEV))
    s_sp, c_sp = hip_ops.absmean_scale(w_sp.to(DEV))
    s_ep, c_ep = hip_ops.absmean_scale(w_ep.to(DEV))
    p_sp = hip_ops.pack_weight(w_sp.to(DEV), s_sp)
    p_ep = hip_ops.pack_weight(w_ep.to(DEV), s_ep)
    y, qy = hip_ops.output_gate(te, cc, p_sp, c_sp, p_ep, c_ep, local.to(DEV), gate.to(DEV), D)
    y_tiled, _ = hip_ops.output_gate(te, cc, p_sp, c_sp, p_ep, c_ep, local.to(DEV), gate.to(DEV), D, quantize=False)
    torch.cuda.synchronize()
    assert torch.equal(y, y_tiled)              # row-complete and tiled kernels agree bit for bit

    def lin(codes, w, s_w, c_w):
        q = hip_ops.unpack_weight(hip_ops.pack_weight(w.to(DEV), s_w), D).cpu().numpy()
        x = codes[0].cpu().numpy()[:, : hip_ops.kpad(D)]
        from hip_helpers import unpermute_layout1
        acc = int_ref.bitlinear_acc(unpermute_layout1(x, D), q).astype(np.float32)
        inv = np.float32(1.0) / codes[1].cpu().numpy().astype(np.float32)
        return torch.from_numpy((acc * inv[:, None]) * np.float32(c_w.cpu()[0])).to(dtype)

    sp = lin(te, w_sp, s_sp, c_sp)
    ep = lin(cc, w_ep, s_ep, c_ep)
    y_ref = local + torch.sigmoid(gate) * sp + ep    # torch ops in dtype, the reference's op order
    err = normwise(to_np(y), to_np(y_ref))
    assert err <= (1e-6 if dtype == torch.float32 else 2 ** -7), err
    qr, sr, rr = hip_ops.quant_act(y)
    assert torch.equal(qy[0], qr) and torch.equal(qy[1], sr) and torch.equal(qy[2], rr)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_output_gate_large_tiles(dtype):
    """The tiled output gate at a shape that takes the 128x256-tile, direct-to-LDS GEMM (d_state 2048
    as in the MIMO layer): both accumulators exact (integer-valued float32 products on the device),
    then the gate in the reference's op order."""
    M, dm, D = 16384, 4096, 2048
    g = torch.Generator().manual_seed(7)
    te_x = torch.tanh(torch.randn(M, D, generator=g)).to(dtype).to(DEV)
    c_x = (torch.randn(M, D, generator=g) * 0.1).to(dtype).to(DEV)
    local = torch.randn(M, dm, generator=g).to(dtype).to(DEV)
    gate = torch.randn(M, dm, generator=g).to(dtype).to(DEV)
    w_sp = (torch.randn(dm, D, generator=g) * 0.02).to(DEV)
    w_ep = (torch.randn(dm, D, generator=g) * 0.02).to(DEV)
    te, cc = _codes(te_x), _codes(c_x)
    s_sp, c_sp = hip_ops.absmean_scale(w_sp)
    s_ep, c_ep = hip_ops.absmean_scale(w_ep)
    p_sp, p_ep = hip_ops.pack_weight(w_sp, s_sp), hip_ops.pack_weight(w_ep, s_ep)
    y, _ = hip_ops.output_gate(te, cc, p_sp, c_sp, p_ep, c_ep, local, gate, D, quantize=False)
    from hip_helpers import unpermute_layout1

    def lin(codes, packed, c_w):
        wq = hip_ops.unpack_weight(packed, D).to(torch.float32)
        xq = torch.from_numpy(unpermute_layout1(codes[0].cpu().numpy()[:, : hip_ops.kpad(D)], D)).to(DEV).float()
        acc = xq @ wq.t().contiguous()                 # exact: |sums| <= 127 * D < 2^24
        return ((acc * (1.0 / codes[1])[:, None]) * c_w[0]).to(dtype)

    y_ref = local + torch.sigmoid(gate) * lin(te, p_sp, c_sp) + lin(cc, p_ep, c_ep)
    err = normwise(to_np(y), to_np(y_ref))
    assert err <= (1e-6 if dtype == torch.float32 else 2 ** -7), err
