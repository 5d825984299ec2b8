"""The SISO decode step with its position in device memory (``tesm_hip_siso_step.step_pos``), captured in
HIP graphs through the C-ABI and replayed, against eager steps of the same layer from the same cache:
bit-identical outputs, states, ring buffers, positions and slots, over ring wrap-around, a partial ring
(prefill shorter than the window), an empty prefill and a global layer (window 0, one-slot ring).

``step_pos = {seq_pos, cache_idx}`` is what makes the step capturable: the decode kernel reads the position
at run time and the step's last launch advances it, so nothing on the host changes between replays
(the form a caller that captures whole decode loops uses).  The eager path itself is checked against the
reference's fixtures and the oracle in test_gpu_decode.py.  Reference step: tesm.py:1274-1400.
"""
import ctypes

import pytest
import torch

from hip_helpers import DEV, need_gpu
from tesm_amd import TESM_SISO, _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _layer(dtype, W, seed):
    torch.manual_seed(seed)
    m = TESM_SISO(d_model=96, d_state=48, ent_rank=16, entanglement_window=W, entanglement_threshold=0.08,
                  decay_init_bias=1.0, max_seq_len=64)
    return m.eval().to(DEV).to(dtype)


def _prefilled(m, u, P, B):
    cache = m.allocate_inference_cache(B, 64)
    ip = {"state_cache": cache}
    with torch.no_grad():
        if P:
            m(u[:, :P], inference_params=ip)
    return ip


class _CapturedSteps:
    """Two graphs of one C-ABI step each (alternating the float64 state buffers), position and slot in
    device memory; the token goes into ``u`` before each replay."""

    def __init__(self, m, ip, max_positions, dtype):
        lib = _lib.load()
        cache = ip["state_cache"]
        kc, vc, state = cache["ent_k_cache"], cache["ent_v_cache"], cache["state"]
        B, D = state.shape
        dev = state.device
        desc, nbytes, self._keep = m._step_plan(B, dtype, dev, kc.dtype, kc.shape[1], False)
        self.u = torch.zeros((B, 1, m.d_model), dtype=dtype, device=dev)
        self.y = torch.empty((B, 1, m.d_model), dtype=dtype, device=dev)
        self.new_state = torch.empty((B, D), dtype=dtype, device=dev)
        self.states = [state.clone(), torch.empty_like(state)]
        self.step_pos = torch.tensor([int(cache["seq_pos"]), int(cache.get("cache_idx", 0))], dtype=torch.int64,
                                     device=dev)
        self.rope = m.rope_table(max_positions, dtype, dev)
        self.ws = torch.empty((max(nbytes, 256),), dtype=torch.uint8, device=dev)
        self.k = 0
        self.graphs = []
        for i in range(2):
            d = _lib.SisoStep()
            ctypes.memmove(ctypes.byref(d), ctypes.byref(desc), ctypes.sizeof(d))
            d.seq_pos, d.cache_idx = 0, 0  # not read: the position comes from step_pos
            d.u, d.ld_u = self.u.data_ptr(), m.d_model
            d.cross_state = None
            d.rope, d.rope_rows = self.rope.data_ptr(), self.rope.shape[0]
            d.state, d.state_out = self.states[i].data_ptr(), self.states[1 - i].data_ptr()
            d.k_cache, d.v_cache = kc.data_ptr(), vc.data_ptr()
            d.y, d.new_state = self.y.data_ptr(), self.new_state.data_ptr()
            d.step_pos = self.step_pos.data_ptr()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, capture_error_mode="relaxed"):
                rc = lib.tesm_hip_siso_decode(ctypes.byref(d), ctypes.c_void_p(self.ws.data_ptr()), self.ws.numel(),
                                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            _lib.check(rc)
            self.graphs.append((g, d))

    def step(self):
        self.graphs[self.k % 2][0].replay()
        self.k += 1
        return self.y

    @property
    def state(self):
        return self.states[self.k % 2]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("P,W,B", [(12, 8, 5), (3, 8, 5), (0, 4, 3), (12, 0, 5), (40, 16, 32)])
def test_captured_steps_match_eager(dtype, P, W, B):
    steps = 11
    m = _layer(dtype, W, seed=7 + P + W)
    gen = torch.Generator().manual_seed(3 + P)
    u = torch.randn(B, P + steps + 1, 96, generator=gen).to(dtype).to(DEV)
    ipa, ipb = _prefilled(m, u, P, B), _prefilled(m, u, P, B)
    eager = []
    with torch.no_grad():
        for s in range(steps):
            y, st = m(u[:, P + s:P + s + 1], inference_params=ipa)
            eager.append((y.clone(), st.clone()))
    gr = _CapturedSteps(m, ipb, P + steps + 1, dtype)
    for s in range(steps):
        gr.u.copy_(u[:, P + s:P + s + 1])
        y = gr.step()
        torch.cuda.synchronize()  # eager work and a synchronisation between replays
        assert torch.equal(y, eager[s][0]), f"step {s}: y"
        assert torch.equal(gr.state, eager[s][1]), f"step {s}: state"
    ca, cb = ipa["state_cache"], ipb["state_cache"]
    pos, idx = (int(v) for v in gr.step_pos.cpu())
    assert (pos, idx) == (ca["seq_pos"], ca["cache_idx"])
    assert torch.equal(cb["ent_k_cache"], ca["ent_k_cache"])
    assert torch.equal(cb["ent_v_cache"], ca["ent_v_cache"])
