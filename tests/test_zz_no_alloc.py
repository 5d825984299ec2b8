"""The allocation-free decode step (tesm_hip_siso_decode_noalloc) against the workspace one
(tesm_hip_siso_decode), through the C-ABI: bit-identical outputs, state and ring buffers, on two
calls in a row, the second with a smaller batch; and the refusal of a step too large for the
library's scratch array."""
import ctypes

import pytest
import torch

from hip_helpers import DEV, need_gpu
from tesm_amd import TESM_SISO, _lib
from tesm_amd.tesm import workspace

pytestmark = pytest.mark.gpu

CFG = dict(d_model=768, d_state=256, ent_rank=64, entanglement_window=16, entanglement_threshold=0.08,
           entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=256)


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _prefilled(m, B, P, dtype, seed):
    u = torch.randn(B, P + 1, CFG["d_model"], generator=torch.Generator().manual_seed(seed)).to(dtype).to(DEV)
    cache = m.allocate_inference_cache(B, P + 1)
    with torch.no_grad():
        m(u[:, :P], inference_params={"state_cache": cache})
    return u, cache


def _step(m, u, cache, noalloc):
    """One decode step through the C-ABI directly; returns (y, state_out, k ring, v ring)."""
    lib = _lib.load()
    B, _, dm = u.shape
    dt = u.dtype
    kc, vc = cache["ent_k_cache"].clone(), cache["ent_v_cache"].clone()
    state = cache["state"].clone()
    desc, nbytes, _keep = m._step_plan(B, dt, u.device, kc.dtype, kc.shape[1], False)
    u2 = u[:, -1, :].contiguous()
    y = torch.empty((B, dm), dtype=dt, device=DEV)
    state_out = torch.empty_like(state)
    rope = m.rope_table(cache["seq_pos"] + 1, dt, u.device)
    desc.seq_pos, desc.cache_idx = cache["seq_pos"], cache["cache_idx"]
    desc.u, desc.ld_u = u2.data_ptr(), dm
    desc.cross_state = None
    desc.rope = rope.data_ptr()
    desc.state, desc.state_out = state.data_ptr(), state_out.data_ptr()
    desc.k_cache, desc.v_cache = kc.data_ptr(), vc.data_ptr()
    desc.y = y.data_ptr()
    desc.new_state = None
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = lib.tesm_hip_siso_decode_noalloc(ctypes.byref(desc), stream)
    else:
        ws = workspace(u.device, nbytes)
        rc = lib.tesm_hip_siso_decode(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return y, state_out, kc, vc


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_decode_matches_workspace_decode(dtype):
    torch.manual_seed(0)
    m = TESM_SISO(**CFG).to(DEV).to(dtype).eval()
    for B, seed in ((32, 1), (5, 2)):          # the second call is smaller
        u, cache = _prefilled(m, B, 40, dtype, seed)
        want = _step(m, u, cache, noalloc=False)
        got = _step(m, u, cache, noalloc=True)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_noalloc_decode_refuses_oversized_step():
    lib = _lib.load()
    torch.manual_seed(0)
    m = TESM_SISO(**CFG).to(DEV).eval()
    B = 4096                                   # codes + in_proj output of 4096 tokens exceed 8 MiB
    desc, nbytes, _keep = m._step_plan(B, torch.float32, torch.device("cuda", 0), torch.float32, 16, False)
    assert nbytes > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.tesm_hip_siso_decode_noalloc(ctypes.byref(desc), None)
    assert rc == 5 and b"scratch" in lib.tesm_hip_last_error()


def test_noalloc_decode_rejects_bad_sizes_before_scratch():
    """A descriptor with out-of-range sizes gets tesm_hip_siso_decode's invalid-argument error, not
    a scratch-size one computed from overflowing products; the workspace query returns -1 for it."""
    lib = _lib.load()
    torch.manual_seed(0)
    m = TESM_SISO(**CFG).to(DEV).eval()
    for field, value in (("B", -3), ("d_model", 1 << 40), ("d_state", 0), ("window", 65)):
        plan, _, _keep = m._step_plan(4, torch.float32, torch.device("cuda", 0), torch.float32, 16, False)
        desc = _lib.SisoStep()  # a copy: the layer keeps its plan
        ctypes.memmove(ctypes.byref(desc), ctypes.byref(plan), ctypes.sizeof(desc))
        setattr(desc, field, value)
        rc = lib.tesm_hip_siso_decode_noalloc(ctypes.byref(desc), None)
        assert rc == 1 and b"siso decode" in lib.tesm_hip_last_error(), (field, rc, lib.tesm_hip_last_error())
        assert lib.tesm_hip_siso_decode_ws_bytes(ctypes.byref(desc)) == -1
