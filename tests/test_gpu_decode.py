"""GPU parity of the TESM_SISO decode path (prefill that fills the ring caches, then one-token steps).

Reference: TESM_SISO.forward cache write (tesm.py:1235-1253), _forward_incremental
(tesm.py:1274-1400), allocate_inference_cache (tesm.py:620-670).  The f32 fixtures were written
by the reference itself; bf16 and larger shapes are checked against the oracle (which restates
the reference, with its bf16 dtype amendment: cache entries cast to the layer dtype).
"""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from flips import check_siso_steps, siso_lockstep
from hip_helpers import DEV, TOL, need_gpu, normwise, to_np
from oracle import tesm_torch as ot
from tesm_amd import TESM_SISO

pytestmark = pytest.mark.gpu

DECODE_F32 = ["decode_f32_prefill", "decode_f32_cross", "decode_f32_empty", "decode_f32_short_prefill"]


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _module(cls, meta, **kw):
    torch.manual_seed(meta["seed"])
    return cls(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=meta["W"],
               entanglement_threshold=0.08, decay_init_bias=1.0, max_seq_len=64, **kw).eval()


def _run(m, u, cs, P, steps, B, dev):
    """Prefill P tokens with a cache, then `steps` single-token steps; returns per-step outputs."""
    cache = m.allocate_inference_cache(B, 64)
    ip = {"state_cache": cache}
    outs = {}
    with torch.no_grad():
        if P:
            outs["prefill_y"] = m(u[:, :P], inference_params=ip,
                                  cross_layer_state=cs[:, :P] if cs is not None else None)[0]
            outs["prefill_state"] = cache["state"].clone()
        for s in range(steps):
            t = P + s
            y, st = m(u[:, t:t + 1], inference_params=ip, cross_layer_state=cs[:, t] if cs is not None else None)
            outs[f"step{s}_y"] = y.clone()
            outs[f"step{s}_state"] = st.clone()
            outs[f"step{s}_kcache"] = cache["ent_k_cache"].clone()
            outs[f"step{s}_vcache"] = cache["ent_v_cache"].clone()
            outs[f"step{s}_cache_idx"] = cache["cache_idx"]
            outs[f"step{s}_seq_pos"] = cache["seq_pos"]
    return outs


@pytest.mark.parametrize("name", DECODE_F32)
def test_decode_vs_reference_fixture(name):
    g, meta = load_golden(name), golden_meta(name)
    m = _module(TESM_SISO, meta).to(DEV)
    u = torch.from_numpy(g["u"]).to(DEV)
    cs = torch.from_numpy(g["cross"]).to(DEV) if "cross" in g else None
    outs = _run(m, u, cs, meta["prefill"], meta["steps"], meta["B"], DEV)
    if meta["prefill"]:
        assert normwise(to_np(outs["prefill_y"]), g["prefill_y"]) <= TOL[torch.float32]
    for s in range(meta["steps"]):
        assert outs[f"step{s}_y"].shape == (meta["B"], 1, meta["dm"])
        assert outs[f"step{s}_state"].dtype == torch.float64
        np.testing.assert_allclose(outs[f"step{s}_state"].cpu().numpy(), g[f"step{s}_state"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(to_np(outs[f"step{s}_kcache"]), g[f"step{s}_kcache"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(to_np(outs[f"step{s}_vcache"]), g[f"step{s}_vcache"], rtol=1e-4, atol=1e-5)
        assert outs[f"step{s}_cache_idx"] == int(g[f"step{s}_cache_idx"])
        assert outs[f"step{s}_seq_pos"] == meta["prefill"] + s + 1
    # outputs: the oracle reproduces these fixtures exactly (tests/test_oracle_fixtures.py); against it,
    # with the device's decisions fed in, every row of every step is within 1e-3
    ref = _module(ot.TESM_SISO, meta)
    m2 = _module(TESM_SISO, meta).to(DEV)
    u_cpu = torch.from_numpy(g["u"])
    cs_cpu = torch.from_numpy(g["cross"]) if "cross" in g else None
    got, want, flips = siso_lockstep(ref, m2, u_cpu, cs_cpu, meta["prefill"], meta["steps"], meta["B"], torch.float32)
    check_siso_steps(got, want, meta["steps"], meta["B"], torch.float32, flips)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("P,steps,W,cross", [(12, 6, 8, False), (3, 9, 8, True), (0, 11, 4, False),
                                             (40, 5, 16, True), (12, 6, 0, False), (0, 7, 0, True)])
def test_decode_random_vs_oracle(dtype, P, steps, W, cross):
    """W = 0 is a global layer: its cache rings hold one slot and its steps add no bias (tesm.py:633,
    1324-1357)."""
    B, dm, D, R = 5, 96, 48, 16
    meta = dict(seed=11 + P + W, dm=dm, D=D, R=R, W=W)
    ref = _module(ot.TESM_SISO, meta).to(dtype)
    m = _module(TESM_SISO, meta).to(DEV).to(dtype)
    gen = torch.Generator().manual_seed(5 + P)
    u = torch.randn(B, P + steps, dm, generator=gen).to(dtype)
    cs = torch.randn(B, P + steps, D, generator=gen).to(dtype) if cross else None
    got, want, flips = siso_lockstep(ref, m, u, cs, P, steps, B, dtype)
    check_siso_steps(got, want, steps, B, dtype, flips)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B", [20, 32])
def test_decode_batch_tiles_vs_oracle(dtype, B):
    """Batches of 17-32 sequences: the in_proj product runs on 32-row tiles with the activation
    quantization inside it."""
    P, steps, W, cross = 12, 4, 8, True
    dm, D, R = 96, 48, 16
    meta = dict(seed=11 + P + W, dm=dm, D=D, R=R, W=W)
    ref = _module(ot.TESM_SISO, meta).to(dtype)
    m = _module(TESM_SISO, meta).to(DEV).to(dtype)
    gen = torch.Generator().manual_seed(5 + P)
    u = torch.randn(B, P + steps, dm, generator=gen).to(dtype)
    cs = torch.randn(B, P + steps, D, generator=gen).to(dtype) if cross else None
    got, want, flips = siso_lockstep(ref, m, u, cs, P, steps, B, dtype)
    check_siso_steps(got, want, steps, B, dtype, flips)


def test_decode_matches_prefill_state_and_cross_state():
    """The float64 state a decode step returns is the cache's; the layer's cross-layer state is
    that state rounded to the layer dtype (tesm.py:1395-1399)."""
    meta = dict(seed=3, dm=64, D=32, R=8, W=8)
    m = _module(TESM_SISO, meta).to(DEV)
    u = torch.randn(2, 10, 64, device=DEV)
    cache = m.allocate_inference_cache(2, 64)
    with torch.no_grad():
        m(u[:, :9], inference_params={"state_cache": cache})
        y, st = m(u[:, 9:], inference_params={"state_cache": cache})
    assert st is cache["state"]
    assert torch.equal(m._last_cross_layer_state, st.to(torch.float32))
    assert cache["seq_pos"] == 10 and cache["cache_idx"] == 1


def test_decode_rejects_bad_cache():
    meta = dict(seed=3, dm=64, D=32, R=8, W=8)
    m = _module(TESM_SISO, meta).to(DEV)
    cache = m.allocate_inference_cache(2, 64)
    cache["ent_k_cache"] = cache["ent_k_cache"][:, :, :4]
    with torch.no_grad(), pytest.raises(RuntimeError, match="inference cache"):
        m(torch.randn(2, 1, 64, device=DEV), inference_params={"state_cache": cache})
