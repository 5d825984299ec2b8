"""GPU parity of the whole TESM_SISO prefill (hip backend) against the reference fixtures and the oracle."""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from flips import assert_unfed, siso_prefill_check
from hip_helpers import DEV, TOL, need_gpu, normwise, to_np
from oracle import tesm_torch as ot
from tesm_amd import TESM_SISO

pytestmark = pytest.mark.gpu

SISO = ["siso_f32", "siso_bf16", "siso_f32_cross_prev", "siso_f32_short", "siso_bf16_cross", "siso_f32_widerank"]


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def build_hip(meta, seed=None):
    torch.manual_seed(meta["seed"] if seed is None else seed)
    return TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=meta["W"],
                     entanglement_threshold=meta["thr"], entanglement_scale=meta["scale"],
                     decay_init_bias=meta["decay_bias"], max_seq_len=max(meta["L"], 64),
                     state_scan_chunk_size=meta["chunk"], entanglement_block_size=meta["block"]).eval()


def build_oracle(meta):
    torch.manual_seed(meta["seed"])
    return ot.TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=meta["W"],
                        entanglement_threshold=meta["thr"], entanglement_scale=meta["scale"],
                        decay_init_bias=meta["decay_bias"], max_seq_len=max(meta["L"], 64),
                        state_scan_chunk_size=meta["chunk"], entanglement_block_size=meta["block"]).eval()


@pytest.mark.parametrize("name", SISO)
def test_siso_prefill_vs_reference_fixture(name):
    g, meta = load_golden(name), golden_meta(name)
    dt = torch.bfloat16 if meta["dtype"] == "torch.bfloat16" else torch.float32
    m = build_hip(meta)
    sd = m.state_dict()
    for k, v in g.items():  # seeded construction reproduces the reference's parameters
        if k.startswith("param/"):
            assert np.array_equal(sd[k[6:]].float().numpy(), v), k
    m = m.to(DEV).to(dt)
    u = torch.from_numpy(g["u"]).to(dt).to(DEV)
    cs = torch.from_numpy(g["cross"]).to(dt).to(DEV) if "cross" in g else None
    h0 = torch.from_numpy(g["h0"]).to(DEV) if "h0" in g else None
    with torch.no_grad():
        y, fin = m(u, cross_layer_state=cs, prev_state=h0)
    torch.cuda.synchronize()
    assert y.shape == u.shape and y.dtype == dt
    assert fin.dtype == torch.float64
    if dt == torch.float32:
        assert normwise(to_np(y), g["y"]) <= TOL[dt]
        np.testing.assert_allclose(fin.cpu().numpy(), g["final_state"], rtol=1e-4, atol=1e-5)
    else:
        # the reference's own bf16 output, nothing fed in: an end-to-end bound on the drift
        assert_unfed(y, torch.from_numpy(g["y"]), name, fin, torch.from_numpy(g["final_state"]))
    states = m._last_cross_layer_state
    assert normwise(to_np(states), g["_parallel_state_scan/out#0"]) <= (1e-5 if dt == torch.float32 else TOL[dt])
    assert m.last_entanglement_map is None
    # against the oracle (which reproduces this fixture exactly on the CPU) with the device's decisions
    # fed in: every row within the north-star tolerance
    ref = build_oracle(meta).to(dt)
    siso_prefill_check(ref, m, torch.from_numpy(g["u"]).to(dt), dt,
                       cs=torch.from_numpy(g["cross"]).to(dt) if "cross" in g else None,
                       h0=torch.from_numpy(g["h0"]) if "h0" in g else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_siso_prefill_random_vs_oracle(dtype):
    cfg = dict(d_model=128, d_state=64, ent_rank=16, entanglement_window=16, entanglement_threshold=0.08,
               entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=512)
    torch.manual_seed(123)
    ref = ot.TESM_SISO(**cfg).eval()
    torch.manual_seed(123)
    m = TESM_SISO(**cfg).eval()
    ref, m = ref.to(dtype), m.to(DEV).to(dtype)
    u = torch.randn(2, 300, 128, generator=torch.Generator().manual_seed(7)).to(dtype)
    y, f, yr, fr = siso_prefill_check(ref, m, u, dtype)
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
    else:
        assert normwise(f.cpu().numpy(), fr.numpy()) <= TOL[dtype]


def test_siso_prefill_properties_at_size():
    """Causality and batch-row independence at a base-like shape (no oracle at full size)."""
    torch.manual_seed(0)
    m = TESM_SISO(d_model=768, d_state=256, ent_rank=64, entanglement_window=16, entanglement_threshold=0.08,
                  entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=2048).to(DEV).to(torch.bfloat16).eval()
    u = torch.randn(4, 1024, 768, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        y, f = m(u)
        y2, f2 = m(u)
        yp, _ = m(u[:, :256])
        yb, fb = m(u[2:3])
    assert torch.equal(y, y2) and torch.equal(f, f2)               # deterministic
    assert torch.equal(y[:, :256], yp)                             # causal: a prefix sees nothing later
    assert torch.equal(y[2:3], yb) and torch.equal(f[2:3], fb)     # rows independent
    assert torch.isfinite(y.float()).all()


def test_gate_out_one_launch_matches_two(monkeypatch):
    """The output gate and out_proj in one launch (bf16, d_model 768, prefills of 4096+ tokens, which take the
    row-complete gate: y's codes stay in the workgroup's LDS) give the same bits as the gate kernel writing
    the codes and a separate out_proj (the path taken with TESM_HIP_NO_GATE_OUT=1, by float32 layers and by
    other widths); tesm.py:1256-1261."""
    from tesm_amd import hip_ops
    torch.manual_seed(3)
    m = TESM_SISO(d_model=768, d_state=256, ent_rank=64, entanglement_window=16, entanglement_threshold=0.08,
                  entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=2048).to(DEV).to(torch.bfloat16).eval()
    u = torch.randn(3, 1500, 768, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        with hip_ops.launch_log() as log:
            y, f = m(u)
        monkeypatch.setenv("TESM_HIP_NO_GATE_OUT", "1")
        with hip_ops.launch_log() as log1:
            y1, f1 = m(u)
    assert any(k.startswith("gate32_kernel<8,3,1,8,24>") for k in log.kernels), log.kernels
    assert not any(k.startswith("mfma32_kernel<1,4,2,1,0,") for k in log.kernels), log.kernels
    assert any(k.startswith("gate32_kernel<8,3,1,8,0>") for k in log1.kernels), log1.kernels
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y, y1) and torch.equal(f, f1)


def test_siso_prefill_errors():
    m = TESM_SISO(d_model=64, d_state=32, ent_rank=8, entanglement_window=8, max_seq_len=16).to(DEV).eval()
    with torch.no_grad():
        with pytest.raises(ValueError, match="exceeds max_seq_len"):
            m(torch.randn(1, 17, 64, device=DEV))
        u0 = torch.randn(1, 0, 64, device=DEV)
        out, fin = m(u0)
        assert out is u0 and fin is None
    with pytest.raises(RuntimeError, match="kernel_backend"):
        m(torch.randn(1, 4, 64, device=DEV))  # grad enabled


def test_siso_prefill_unfused_fallbacks_vs_oracle():
    """d_model > 1024 and d_state > 512 take the unfused output-gate and entanglement paths."""
    cfg = dict(d_model=1100, d_state=520, ent_rank=8, entanglement_window=4, entanglement_threshold=0.08,
               entanglement_scale=0.2, decay_init_bias=1.0, max_seq_len=64)
    torch.manual_seed(5)
    ref = ot.TESM_SISO(**cfg).eval()
    torch.manual_seed(5)
    m = TESM_SISO(**cfg).to(DEV).eval()
    u = torch.randn(1, 20, 1100, generator=torch.Generator().manual_seed(3))
    y, f, yr, fr = siso_prefill_check(ref, m, u, torch.float32)
    np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
