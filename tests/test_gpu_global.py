"""GPU parity of global causal entanglement (entanglement_window = 0): TESM_SISO (tesm.py:963-1063,
torch branch 1040-1052) against the reference's fixture and the oracle, and TESMMIMO_Optimized's
global branch (tesm_mimo.py:590-687) and its sampled statistics (:469-482) against the oracle."""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from flips import Flips, Taps, assert_rows, install, uninstall
from hip_helpers import DEV, TOL, need_gpu, normwise, to_np
from oracle import tesm_torch as ot
from tesm_amd import TESM_SISO, TESMMIMO_Optimized

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def test_siso_global_vs_reference_fixture():
    g, meta = load_golden("siso_global_f32"), golden_meta("siso_global_f32")
    torch.manual_seed(meta["seed"])
    m = TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=0,
                  entanglement_threshold=0.08, max_seq_len=64).eval()
    sd = m.state_dict()
    for k, v in g.items():  # seeded construction reproduces the reference's parameters
        if k.startswith("param/"):
            assert np.array_equal(sd[k[6:]].float().numpy(), v), k
    m = m.to(DEV)
    torch.manual_seed(meta["seed"])
    ref = ot.TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=0,
                       entanglement_threshold=0.08, max_seq_len=64).eval()
    u = torch.from_numpy(g["u"])
    y, fin, _ = _siso_lockstep(ref, m, u, None, torch.float32)
    assert normwise(to_np(y), g["y"]) <= TOL[torch.float32]
    np.testing.assert_allclose(fin.cpu().numpy(), g["final_state"], rtol=1e-5, atol=1e-6)
    assert m.last_entanglement_map is None  # as the reference's fast (CUDA) path


def _siso_lockstep(ref, m, u, cs, dtype):
    """One global-entanglement prefill on the device (decision taps on) and on the oracle with the
    device's codes and ternary decisions fed in (near-ties only, checked); every row of y within the
    north-star tolerance.  Returns (y, final state, oracle final state)."""
    B, L, dm = u.shape
    D = m.d_state
    flips = Flips(dtype)
    with torch.no_grad():
        with Taps(B * L, D, dm, DEV, (B, L, (L + 63) // 64 * 64), d_state=D, dtype=dtype) as tp:
            y, f = m(u.to(DEV), cross_layer_state=cs.to(DEV) if cs is not None else None)
        install(ref, flips, tp, "global", states=m._last_cross_layer_state)
        yr, fr = ref(u, cross_layer_state=cs)
        uninstall(ref)
    assert_rows(to_np(y), to_np(yr), dtype, f"global prefill ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    assert flips.tern_flips <= max(4, 0.01 * flips.terns), flips.summary()
    return y, f, fr


def _siso(cls, seed, dtype, **kw):
    cfg = dict(d_model=96, d_state=48, ent_rank=16, entanglement_window=0, entanglement_threshold=0.05,
               entanglement_scale=0.3, decay_init_bias=2.0, max_seq_len=512)
    cfg.update(kw)
    torch.manual_seed(seed)
    m = cls(**cfg).eval()
    with torch.no_grad():  # a non-trivial relative-position bias
        gg = torch.Generator().manual_seed(seed + 1)
        m.global_rel_pos_embed.copy_(torch.randn(m.global_rel_pos_embed.shape, generator=gg) * 0.05)
        m.global_rel_pos_scale.fill_(1.5)
        m.global_rel_pos_bias.fill_(-0.01)
    return m.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,cross", [(2, 100, False), (1, 300, True), (3, 7, False)])
def test_siso_global_random_vs_oracle(dtype, B, L, cross):
    """L = 300 in bf16 runs past 256, where the reference's bf16 positions (arange in the layer
    dtype) are rounded and the bias becomes a function of the rounded difference."""
    ref = _siso(ot.TESM_SISO, 11 + L, dtype)
    m = _siso(TESM_SISO, 11 + L, dtype).to(DEV)
    gen = torch.Generator().manual_seed(L)
    u = torch.randn(B, L, 96, generator=gen).to(dtype)
    cs = torch.randn(B, L, 48, generator=gen).to(dtype) if cross else None
    y, f, fr = _siso_lockstep(ref, m, u, cs, dtype)
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
    else:
        assert normwise(f.cpu().numpy(), fr.numpy()) <= TOL[dtype]


def test_siso_global_prefill_fills_cache():
    """With window 0 the reference allocates one-slot rings (tesm.py:620-670) and the prefill stores the
    last key and state there (tesm.py:1240-1252)."""
    ref = _siso(ot.TESM_SISO, 5, torch.float32)
    m = _siso(TESM_SISO, 5, torch.float32).to(DEV)
    u = torch.randn(2, 20, 96, generator=torch.Generator().manual_seed(2))
    cr, cm = ref.allocate_inference_cache(2, 64), m.allocate_inference_cache(2, 64)
    with torch.no_grad():
        ref(u, inference_params={"state_cache": cr})
        m(u.to(DEV), inference_params={"state_cache": cm})
    for k in ("ent_k_cache", "ent_v_cache"):
        assert cm[k].shape == cr[k].shape == (2, 1, cr[k].shape[2])
        np.testing.assert_allclose(to_np(cm[k]), cr[k].numpy(), rtol=1e-4, atol=1e-5)
    assert cm["seq_pos"] == 20 and cm["cache_idx"] == 0


def _mimo(cls, seed, dtype):
    torch.manual_seed(seed)
    m = cls(d_model=64, d_state=16, n_heads=2, mimo_rank=3, ent_rank=8, entanglement_window=0,
            entanglement_threshold=0.05, entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=512).eval()
    with torch.no_grad():
        gg = torch.Generator().manual_seed(seed + 7)
        m.mimo_x.copy_(torch.rand(m.mimo_x.shape, generator=gg) + 0.25)
        m.mimo_o.copy_(torch.rand(m.mimo_o.shape, generator=gg) + 0.25)
        m.global_rel_pos_embed.copy_(torch.randn(m.global_rel_pos_embed.shape, generator=gg) * 0.05)
    return m.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L", [(2, 70, ), (1, 33), (2, 5)])
def test_mimo_global_random_vs_oracle(dtype, B, L):
    ref = _mimo(ot.TESMMIMO_Optimized, L, dtype)
    m = _mimo(TESMMIMO_Optimized, L, dtype).to(DEV)
    u = torch.randn(B, L, 64, generator=torch.Generator().manual_seed(3)).to(dtype)
    flips = Flips(dtype)
    with torch.no_grad():
        with Taps(B * L, 32, 64, DEV, (B, L, (L + 63) // 64 * 64), states=True, dtype=dtype) as tp:
            y, f = m(u.to(DEV))
        install(ref, flips, tp, "global", states=tp.S)
        yr, fr = ref(u)
        uninstall(ref)
        # the statistics below come from an untapped oracle run
        ref(u)
    assert_rows(to_np(y), to_np(yr), dtype, f"mimo global prefill ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    assert flips.tern_flips <= max(4, 0.01 * flips.terns), flips.summary()
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
    else:
        assert normwise(f.cpu().numpy(), fr.numpy()) <= TOL[dtype]
    # sampled statistics of the global branch: (B, S, S) over S = min(L, 32), no mask, no bias
    want, got = ref._stats_ternary_buffer, m._stats_ternary_buffer
    S = min(L, 32)
    assert got.shape == want.shape == (B * S * S,)
    diff = (got.cpu() != want).float().mean().item()
    assert diff <= (0.002 if dtype == torch.float32 else 0.01), diff
    a, b = m.last_entanglement_stats, ref.last_entanglement_stats
    for k in a:
        assert abs(a[k] - b[k]) <= diff + 1e-12
