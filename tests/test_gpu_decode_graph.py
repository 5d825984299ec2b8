"""Graph-replayed decode steps (SisoDecodeGraph: the step position in device memory, two captured
graphs alternating the state buffers) against eager steps of the same layer from the same cache:
bit-identical outputs, states, ring buffers, positions and slots, over ring wrap-around, a partial
ring (prefill shorter than the window), an empty prefill and a global layer (window 0, one-slot ring).
The eager path itself is checked against the reference's fixtures and the oracle in
test_gpu_decode.py; this file pins the replay to it.  Reference step: tesm.py:1274-1400.
"""
import pytest
import torch

from hip_helpers import DEV, need_gpu
from tesm_amd import SisoDecodeGraph, TESM_SISO

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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("P,W,B", [(12, 8, 5), (3, 8, 5), (0, 4, 3), (12, 0, 5), (40, 16, 32)])
def test_graph_steps_match_eager(dtype, P, W, B):
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
    gr = SisoDecodeGraph(m, ipb, max_positions=P + steps + 1, dtype=dtype)
    for s in range(steps):
        gr.u.copy_(u[:, P + s:P + s + 1])
        y = gr.step()
        torch.cuda.synchronize()
        assert torch.equal(y, eager[s][0]), f"step {s}: y"
        assert torch.equal(gr.state, eager[s][1]), f"step {s}: state"
    gr.sync_cache()
    ca, cb = ipa["state_cache"], ipb["state_cache"]
    assert (cb["seq_pos"], cb["cache_idx"]) == (ca["seq_pos"], ca["cache_idx"])
    assert torch.equal(cb["ent_k_cache"], ca["ent_k_cache"])
    assert torch.equal(cb["ent_v_cache"], ca["ent_v_cache"])
    with torch.no_grad():  # eager steps continue from the handed-back cache
        ya, _ = m(u[:, -1:], inference_params=ipa)
        yb, _ = m(u[:, -1:], inference_params=ipb)
    assert torch.equal(ya, yb)


def test_graph_rejects_short_rope_table():
    m = _layer(torch.float32, 8, seed=1)
    u = torch.randn(2, 5, 96, device=DEV)
    ip = _prefilled(m, u, 4, 2)
    with pytest.raises(ValueError):
        SisoDecodeGraph(m, ip, max_positions=4)


def test_graph_refuses_steps_past_table_and_stale_weights():
    """A replay whose position would pass the RoPE table, or after the layer's weights changed, raises
    instead of returning wrong outputs (the graphs hold the table and packed weights of capture)."""
    m = _layer(torch.float32, 8, seed=2)
    u = torch.randn(2, 10, 96, device=DEV)
    ip = _prefilled(m, u, 6, 2)
    gr = SisoDecodeGraph(m, ip, max_positions=8)   # positions 6 and 7 fit
    for s in range(2):
        gr.u.copy_(u[:, 6 + s:7 + s])
        gr.step()
    with pytest.raises(RuntimeError, match="past the RoPE table"):
        gr.step()
    ip2 = _prefilled(m, u, 6, 2)
    gr2 = SisoDecodeGraph(m, ip2, max_positions=16)
    gr2.u.copy_(u[:, 6:7])
    gr2.step()
    with torch.no_grad():
        m.out_proj.weight.mul_(2.0)                # an in-place update bumps the weight version
    with pytest.raises(RuntimeError, match="changed after capture"):
        gr2.step()
    torch.cuda.synchronize()
