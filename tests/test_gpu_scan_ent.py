"""GPU parity of the state scan, the RoPE table and the local-window entanglement against the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from hip_helpers import DEV, TOL, need_gpu, normwise, to_np
from oracle import tesm_torch as ot
from tesm_amd import hip_ops

pytestmark = pytest.mark.gpu

SISO = ["siso_f32", "siso_bf16", "siso_f32_cross_prev", "siso_f32_short", "siso_bf16_cross", "siso_f32_widerank"]


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _dt(meta):
    return torch.bfloat16 if meta["dtype"] == "torch.bfloat16" else torch.float32


def _oracle_module(C, cs, W=8, R=8):
    return ot.TESM_SISO(d_model=8, d_state=C, ent_rank=R, entanglement_window=W, state_scan_chunk_size=cs).eval()


# -- scan ----------------------------------------------------------------------------------
@pytest.mark.parametrize("name", SISO)
def test_scan_vs_reference_stage(name):
    g, meta = load_golden(name), golden_meta(name)
    dt = _dt(meta)
    d = torch.from_numpy(g["_parallel_state_scan/arg0#0"]).to(dt).to(DEV)
    u = torch.from_numpy(g["_parallel_state_scan/arg1#0"]).to(dt).to(DEV)
    h0 = torch.from_numpy(g["h0"]).to(DEV) if "h0" in g else None
    states, h_final = hip_ops.scan(d, u, meta["chunk"], h0=h0)
    ref = g["_parallel_state_scan/out#0"]
    tol = 1e-5 if dt == torch.float32 else 2 ** -8
    assert normwise(to_np(states), ref) <= tol
    if dt == torch.float32:
        np.testing.assert_allclose(h_final.cpu().numpy(), g["final_state"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,C,cs", [(2, 1000, 96, 16), (3, 77, 40, 8), (1, 5, 16, 16), (2, 300, 64, 32),
                                      (1, 64, 8, 1), (2, 129, 33, 7)])
def test_scan_random_vs_oracle(dtype, B, L, C, cs):
    g = torch.Generator().manual_seed(B * L + C + cs)
    decay = torch.sigmoid(torch.randn(B, L, C, generator=g)).to(dtype)
    update = (torch.sigmoid(torch.randn(B, L, C, generator=g)) * torch.tanh(torch.randn(B, L, C, generator=g))).to(dtype)
    h0 = torch.randn(B, C, generator=g, dtype=torch.float64)
    m = _oracle_module(C, cs)
    with torch.no_grad():
        ref = m._parallel_state_scan(decay, update, prev_state=h0)
    states, h_final = hip_ops.scan(decay.to(DEV), update.to(DEV), cs, h0=h0.to(DEV))
    tol = 1e-5 if dtype == torch.float32 else 2 ** -8
    assert normwise(to_np(states), to_np(ref)) <= tol
    np.testing.assert_allclose(h_final.cpu().numpy(), m._last_scan_state_f64.numpy(), rtol=1e-4, atol=1e-5)


def _scan_inputs(B, L, C, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    decay = torch.sigmoid(torch.randn(B, L, C, generator=g) + 2.0).to(dtype)
    update = (torch.sigmoid(torch.randn(B, L, C, generator=g)) * torch.tanh(torch.randn(B, L, C, generator=g))).to(dtype)
    h0 = torch.randn(B, C, generator=g, dtype=torch.float64)
    return decay, update, h0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,C,cs", [(2, 5000, 300, 16), (1, 4097, 520, 8), (3, 2048, 256, 16)])
def test_scan_lookback_many_spans_vs_oracle(dtype, B, L, C, cs):
    """Long sequences (more than 64 spans of 32 positions: the look-back walks several windows) and
    several 256-channel groups per row; decays near 1 carry the state across many spans."""
    decay, update, h0 = _scan_inputs(B, L, C, dtype, B * L + C)
    m = _oracle_module(C, cs)
    with torch.no_grad():
        ref = m._parallel_state_scan(decay, update, prev_state=h0)
    states, h_final = hip_ops.scan(decay.to(DEV), update.to(DEV), cs, h0=h0.to(DEV))
    # bf16: states reach [1, 2) here, where one bf16 step of the output rounding is 2^-7 of the value
    tol = 1e-5 if dtype == torch.float32 else 2 ** -7
    assert normwise(to_np(states), to_np(ref)) <= tol
    np.testing.assert_allclose(h_final.cpu().numpy(), m._last_scan_state_f64.numpy(), rtol=1e-4, atol=1e-5)


def _scan_abi(decay, update, cs, h0, ws, nbytes):
    """tesm_hip_scan through the C-ABI with a caller-chosen workspace pointer."""
    from tesm_amd import _lib
    from tesm_amd.hip_ops import _p, _stream, dt_code
    lib = _lib.load()
    B, L, C = decay.shape
    states = torch.empty_like(decay)
    h_final = torch.empty((B, C), dtype=torch.float64, device=decay.device)
    _lib.check(lib.tesm_hip_scan(_p(decay), C, _p(update), C, dt_code(decay.dtype), B, L, C, cs, _p(h0), _p(states), C,
                                 dt_code(decay.dtype), _p(h_final), ctypes.c_void_p(ws), nbytes, _stream(decay)))
    return states, h_final


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_workspace_reuse_and_three_pass_path(dtype):
    """One workspace across calls of different sizes (the look-back flags are cleared per call), and the
    three-pass path (taken for a workspace that is not 8-byte aligned) against the same oracle."""
    from tesm_amd import _lib
    lib = _lib.load()
    cs = 16
    shapes = [(2, 3000, 300), (1, 700, 64), (2, 3000, 300)]
    nbytes = max(int(lib.tesm_hip_scan_ws_bytes(B, L, C, cs)) for B, L, C in shapes)
    ws = torch.full((nbytes + 4,), 0x7f, dtype=torch.uint8, device=DEV)  # stale bytes in the flag region
    for i, (B, L, C) in enumerate(shapes):
        decay, update, h0 = _scan_inputs(B, L, C, dtype, 100 + i)
        m = _oracle_module(C, cs)
        with torch.no_grad():
            ref = m._parallel_state_scan(decay, update, prev_state=h0)
        d, u, h = decay.to(DEV), update.to(DEV), h0.to(DEV)
        tol = 1e-5 if dtype == torch.float32 else 2 ** -7  # one bf16 step of the output rounding
        for offset in (0, 4):
            states, h_final = _scan_abi(d, u, cs, h, ws.data_ptr() + offset, nbytes)
            torch.cuda.synchronize()
            assert normwise(to_np(states), to_np(ref)) <= tol, (B, L, C, offset)
            np.testing.assert_allclose(h_final.cpu().numpy(), m._last_scan_state_f64.numpy(), rtol=1e-4, atol=1e-5)


def test_scan_reproduces_closed_form_clamp():
    """Small decays drive the within-chunk product below 1e-12, where the reference's closed form
    (tesm.py:1085-1088) departs from the plain recurrence; the kernel follows the reference."""
    B, L, C, cs = 1, 64, 16, 16
    g = torch.Generator().manual_seed(11)
    decay = torch.full((B, L, C), 0.05) * torch.rand(B, L, C, generator=g) + 0.01
    update = torch.randn(B, L, C, generator=g)
    m = _oracle_module(C, cs)
    with torch.no_grad():
        ref = m._parallel_state_scan(decay, update)
    plain = torch.zeros(B, C, dtype=torch.float64)
    rec = []
    for t in range(L):
        plain = decay[:, t].double() * plain + update[:, t].double()
        rec.append(plain.clone())
    rec = torch.stack(rec, 1)
    assert normwise(rec.numpy(), ref.double().numpy()) > 1e-3   # the clamp matters here
    states, _ = hip_ops.scan(decay.to(DEV), update.to(DEV), cs)
    assert normwise(to_np(states), ref.numpy()) <= 1e-5


def test_scan_invariants():
    """decay == 1 gives a prefix sum; linearity in the update."""
    B, L, C = 2, 513, 24
    g = torch.Generator().manual_seed(5)
    u = torch.randn(B, L, C, generator=g)
    s, _ = hip_ops.scan(torch.ones(B, L, C, device=DEV), u.to(DEV), 16)
    assert normwise(to_np(s), torch.cumsum(u.double(), 1).numpy()) <= 1e-5
    d = torch.sigmoid(torch.randn(B, L, C, generator=g)).to(DEV)
    u2 = torch.randn(B, L, C, generator=g).to(DEV)
    s1, _ = hip_ops.scan(d, u.to(DEV), 16)
    s2, _ = hip_ops.scan(d, u2, 16)
    s12, _ = hip_ops.scan(d, 2.0 * u.to(DEV) - u2, 16)
    assert normwise(to_np(s12), to_np(2.0 * s1 - s2)) <= 1e-5


# -- RoPE table ----------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L,R", [(40, 8), (2048, 64), (512, 48)])
def test_rope_table_vs_oracle(dtype, L, R):
    tab = hip_ops.rope_table(L, R, dtype, DEV).cpu()
    half = R // 2
    pos = torch.arange(0, L, dtype=torch.float32)
    idx = torch.arange(half, dtype=torch.float32)
    theta = pos.unsqueeze(1) * (1.0 / (10000.0 ** (2.0 * idx / R)))
    c, s = theta.cos().to(dtype).float(), theta.sin().to(dtype).float()
    # torch's CPU cos/sin are within one ulp of the correctly rounded values the kernel produces
    ulp = torch.finfo(dtype).eps
    assert torch.all((tab[..., 0] - c).abs() <= ulp * c.abs().clamp_min(2 ** -20) + 1e-30)
    assert torch.all((tab[..., 1] - s).abs() <= ulp * s.abs().clamp_min(2 ** -20) + 1e-30)
    assert (tab[..., 0] == c).float().mean() > 0.9


# -- local entanglement ---------------------------------------------------------------------
def _identity_rope(L, R):
    t = torch.zeros(L, R // 2, 2, device=DEV)
    t[..., 0] = 1.0
    return t


def _siso_params(g):
    return torch.from_numpy(g["param/local_entanglement_bias"])


@pytest.mark.parametrize("name", SISO)
def test_local_ent_vs_reference_stage(name):
    """Kernel fed the reference's own post-RoPE q, k and states (identity RoPE table)."""
    g, meta = load_golden(name), golden_meta(name)
    dt = _dt(meta)
    q = torch.from_numpy(g["_compute_entanglement/arg0#0"]).to(dt).to(DEV)
    k = torch.from_numpy(g["_compute_entanglement/arg1#0"]).to(dt).to(DEV)
    S = torch.from_numpy(g["_compute_entanglement/arg2#0"]).to(dt).to(DEV)
    B, L, R = q.shape
    W = min(meta["W"], L)
    bias = _siso_params(g)[-W:]
    out = hip_ops.local_ent(q, k, _identity_rope(L, R), S, bias, W, meta["thr"], meta["scale"],
                            outputs=("avg", "e", "c", "e_tanh"), want_tern=True)
    tern = out["tern"].cpu().numpy()[:, :, 0, :]
    assert np.array_equal(tern, g["last_map"].astype(np.int8))
    ref = g["_compute_entanglement/out#0"]
    assert normwise(to_np(out["avg"]), ref) <= (1e-6 if dt == torch.float32 else 2 ** -8)
    Sref = torch.from_numpy(g["_compute_entanglement/arg2#0"]).to(dt)
    e_ref = Sref + meta["scale"] * (torch.from_numpy(ref).to(dt) - Sref)
    assert normwise(to_np(out["e"]), to_np(e_ref)) <= (1e-6 if dt == torch.float32 else 2 ** -8)
    assert normwise(to_np(out["c"]), to_np(e_ref - Sref)) <= (1e-6 if dt == torch.float32 else 2 ** -7)
    assert normwise(to_np(out["e_tanh"]), to_np(torch.tanh(e_ref))) <= (1e-6 if dt == torch.float32 else 2 ** -7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,R,D,W", [(2, 300, 16, 64, 16), (1, 70, 64, 96, 32), (3, 9, 8, 16, 16),
                                       (1, 200, 48, 130, 64)])
def test_local_ent_random_vs_oracle(dtype, B, L, R, D, W):
    """Raw q/k with the kernel's RoPE table against the oracle's RoPE + entanglement."""
    g = torch.Generator().manual_seed(B + L + R + D + W)
    m = ot.TESM_SISO(d_model=8, d_state=D, ent_rank=R, entanglement_window=W, entanglement_threshold=0.08,
                     max_seq_len=max(L, 64)).eval()
    with torch.no_grad():
        m.local_entanglement_bias.copy_(torch.randn(W, generator=g) * 0.3)
    m = m.to(dtype)
    q = torch.randn(B, L, R, generator=g).to(dtype)
    k = torch.randn(B, L, R, generator=g).to(dtype)
    S = torch.randn(B, L, D, generator=g).to(dtype)
    with torch.no_grad():
        ref = m._compute_entanglement(m._apply_rope(q), m._apply_rope(k), S)
    rope = hip_ops.rope_table(L, R, dtype, DEV)
    out = hip_ops.local_ent(q.to(DEV), k.to(DEV), rope, S.to(DEV), m.local_entanglement_bias.detach()[-min(W, L):],
                            min(W, L), 0.08, 0.2, outputs=("avg",), want_tern=True)
    tern = out["tern"].cpu().numpy()[:, :, 0, :]
    ref_map = m.last_entanglement_map.float().numpy().astype(np.int8)
    agree = (tern == ref_map).mean()
    assert agree >= 0.999, agree                  # RoPE cos/sin may differ by an ulp -> rare threshold flips
    rows_equal = (tern == ref_map).all(-1)
    a, r = to_np(out["avg"]), to_np(ref)
    assert normwise(a[rows_equal], r[rows_equal]) <= (1e-5 if dtype == torch.float32 else 2 ** -7)


def test_local_ent_cross_bias_and_thresholds():
    """q_add is added after RoPE (tesm.py:1209-1218); all-|score| <= thr rows give zero output."""
    B, L, R, D, W = 2, 50, 8, 16, 8
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, L, R, generator=g)
    k = torch.randn(B, L, R, generator=g)
    S = torch.randn(B, L, D, generator=g)
    cq = torch.randn(B, L, R, generator=g)
    m = ot.TESM_SISO(d_model=8, d_state=D, ent_rank=R, entanglement_window=W, entanglement_threshold=0.08).eval()
    with torch.no_grad():
        ref = m._compute_entanglement(m._apply_rope(q) + cq, m._apply_rope(k), S)
    rope = hip_ops.rope_table(L, R, torch.float32, DEV)
    bias = m.local_entanglement_bias.detach()
    out = hip_ops.local_ent(q.to(DEV), k.to(DEV), rope, S.to(DEV), bias, W, 0.08, 0.2, q_add=cq.to(DEV))
    assert normwise(to_np(out["avg"]), ref.numpy()) <= 1e-4
    # huge threshold: every ternary weight is 0 -> avg == 0
    out0 = hip_ops.local_ent(q.to(DEV), k.to(DEV), rope, S.to(DEV), bias, W, 1e9, 0.2)
    assert float(out0["avg"].abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_local_ent_prerounded_bias(dtype):
    """A bias already in window_bias() form (float32, rounded to the layer dtype; what the bench's isolated
    ops pass, so a call launches no conversion) gives the same bits as the raw bias, with and without codes."""
    B, L, R, D, W = 2, 70, 16, 64, 16
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, L, R, generator=g).to(dtype).to(DEV)
    k = torch.randn(B, L, R, generator=g).to(dtype).to(DEV)
    S = torch.randn(B, L, D, generator=g).to(dtype).to(DEV)
    bias = torch.randn(W, generator=g) * 0.3
    rope = hip_ops.rope_table(L, R, dtype, DEV)
    ready = hip_ops.window_bias(bias, 1, W, dtype, S.device)
    a = hip_ops.local_ent(q, k, rope, S, bias, W, 0.08, 0.2, outputs=("avg", "c"))
    b = hip_ops.local_ent(q, k, rope, S, ready, W, 0.08, 0.2, outputs=("avg", "c"), bias_rounded=True)
    assert torch.equal(a["avg"], b["avg"]) and torch.equal(a["c"], b["c"])
    qa = hip_ops.local_ent_quant(q, k, rope, S, bias, W, 0.08, 0.2)
    qb = hip_ops.local_ent_quant(q, k, rope, S, ready, W, 0.08, 0.2, bias_rounded=True)
    for name in ("te", "c"):
        for x, y in zip(qa[name], qb[name]):
            assert torch.equal(x, y), name
    for bad in (bias, ready.to(torch.float64), ready.reshape(W, 1).t().contiguous()[:, : W - 1]):
        with pytest.raises(ValueError):  # not window_bias()'s form: host memory, float64, wrong size
            hip_ops.local_ent(q, k, rope, S, bad, W, 0.08, 0.2, bias_rounded=True)
