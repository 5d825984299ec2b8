"""GPU parity of the block and model around the layers: RMSNorm (block.py:7-16), FeedForward
(mixer_seq_simple.py:25-67), Block (block.py:19-47) and TESMLMHeadModel (mixer_seq_simple.py:69-345),
against the oracle and the reference's own tiny() model fixture."""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from flips import Flips, ModelTaps, Taps, assert_rows, install_ffn, uninstall
from hip_helpers import DEV, TOL, bf16_bits, need_gpu, normwise, to_np, unpermute_layout1
from oracle import int_ref
from oracle import tesm_torch as ot
from tesm_amd import Block, FeedForward, RMSNorm, TESMConfig, TESMLMHeadModel, TESM_SISO, hip_ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _small_cfg(**kw):
    base = dict(d_model=128, n_layer=2, d_intermediate=320, vocab_size=500, max_seq_len=96, d_state=32, ent_rank=16,
                entanglement_window=8, entanglement_threshold=0.05, decay_init_bias=1.0, tie_embeddings=True)
    base.update(kw)
    return TESMConfig(**base)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("res", [None, torch.float32, "same"])
@pytest.mark.parametrize("M,D", [(7, 128), (33, 768), (4, 4100)])
def test_rmsnorm_vs_oracle(dtype, res, M, D):
    g = torch.Generator().manual_seed(M + D)
    x = (torch.randn(M, D, generator=g) * 2).to(dtype)
    r = None
    if res is not None:
        r = torch.randn(M, D, generator=g).to(dtype if res == "same" else res)
    ref = ot.RMSNorm(D, eps=1e-5)
    with torch.no_grad():
        ref.weight.copy_(torch.rand(D, generator=g) + 0.5)
    ref = ref.to(dtype)
    m = RMSNorm(D, eps=1e-5).to(DEV).to(dtype)
    with torch.no_grad():
        m.weight.copy_(ref.weight)
        s_ref = x + r if r is not None else x
        y_ref = ref(s_ref.to(dtype))
        y, s_out, codes = m.fused(x.to(DEV), r.to(DEV) if r is not None else None,
                                  residual_dtype=s_ref.dtype, codes_eps=1e-5)
    # the add and its dtype are exact; the norm agrees but for the float order of the mean.  In bf16
    # torch's CPU rsqrt rounds sqrt to bf16 before the reciprocal for the elements of a (M, 1) tensor
    # outside its 32-wide vector chunks (here every row when M < 32), while the kernel takes
    # 1/sqrt in float (the vector chunks' result): a row's scale may then differ by one bf16 ulp.
    assert s_out.dtype == s_ref.dtype and torch.equal(s_out.cpu(), s_ref)
    tol = 2e-6 if dtype == torch.float32 else 1e-2
    assert normwise(to_np(y), to_np(y_ref)) <= tol
    # the fused codes are those of quant_act on the kernel's own y
    q, s, rs = codes
    if dtype == torch.bfloat16:
        q_ref, sc_ref = int_ref.quant_act(bf16_bits(y), bf16_bits=True)
    else:
        q_ref, sc_ref = int_ref.quant_act(y.cpu().numpy())
    assert np.array_equal(unpermute_layout1(q.cpu().numpy(), D), q_ref)
    assert np.array_equal(s.cpu().numpy(), sc_ref)
    assert np.array_equal(rs.cpu().numpy(), q_ref.astype(np.int64).sum(1))
    assert np.all(unpermute_layout1(q.cpu().numpy(), q.shape[1])[:, D:] == 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 3, 20, 32, 300])
def test_ffn_vs_oracle(dtype, M):
    cfg = _small_cfg()
    torch.manual_seed(M)
    ref = ot.FeedForward(cfg).eval().to(dtype)
    torch.manual_seed(M)
    m = FeedForward(cfg).to(DEV).to(dtype).eval()
    x = torch.randn(M, cfg.d_model, generator=torch.Generator().manual_seed(3)).to(dtype)
    flips = Flips(dtype)
    with torch.no_grad():
        with Taps(M, 1, cfg.d_model, DEV, d_inter=cfg.d_intermediate, dtype=dtype) as tp:
            y = m(x.to(DEV))
        # the codes path (as after norm2) gives the same bits
        q, s, rs = hip_ops.quant_act(x.to(DEV), m.gate_proj.bit_eps)
        y2 = m.forward_codes((q, s, rs), x.shape)
        install_ffn(ref, flips, tp)
        y_ref = ref(x)
        uninstall(ref)
    assert torch.equal(y, y2)
    assert_rows(to_np(y), to_np(y_ref), dtype, f"ffn ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()


def test_ffn_swiglu_large_tiles():
    """The prefill-size product (32x32 MFMA tiles) against the split-K decode path, row for row."""
    cfg = _small_cfg(d_model=768, d_intermediate=2048)
    torch.manual_seed(5)
    m = FeedForward(cfg).to(DEV).to(torch.bfloat16).eval()
    x = torch.randn(1024, 768, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        y = m(x)
        y_rows = torch.cat([m(x[i:i + 16]) for i in range(0, 64, 16)])
    assert torch.equal(y[:64], y_rows)


def _block_pair(dtype, cfg):
    def mixer(cls):
        return lambda dim: cls(d_model=dim, d_state=cfg.d_state, ent_rank=cfg.ent_rank,
                               entanglement_window=cfg.entanglement_window,
                               entanglement_threshold=cfg.entanglement_threshold,
                               decay_init_bias=cfg.decay_init_bias, max_seq_len=cfg.max_seq_len)
    torch.manual_seed(21)
    ref = ot.Block(cfg.d_model, mixer(ot.TESM_SISO), lambda d: ot.FeedForward(cfg), eps=cfg.norm_epsilon,
                   residual_in_fp32=True).eval()
    torch.manual_seed(21)
    m = Block(cfg.d_model, mixer(TESM_SISO), lambda d: FeedForward(cfg), residual_in_fp32=True).eval()
    with torch.no_grad():
        for mod in (ref, m):
            mod.norm.weight.copy_(torch.linspace(0.5, 1.5, cfg.d_model))
            mod.norm2.weight.copy_(torch.linspace(1.5, 0.5, cfg.d_model))
    return ref.to(dtype), m.to(DEV).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("first", [True, False])
def test_block_vs_oracle(dtype, first):
    cfg = _small_cfg()
    ref, m = _block_pair(dtype, cfg)
    g = torch.Generator().manual_seed(8)
    h = torch.randn(2, 40, cfg.d_model, generator=g).to(dtype)
    res = None if first else torch.randn(2, 40, cfg.d_model, generator=g)
    flips = Flips(dtype)
    mt = ModelTaps([m], 2, 40)
    with torch.no_grad():
        y, r, f = m(h.to(DEV), res.to(DEV) if res is not None else None)
        mt.restore()
        mt.install([ref], flips)
        yr, rr, fr = ref(h, res)
        uninstall(ref)
    assert r.dtype == torch.float32 and rr.dtype == torch.float32
    assert y.dtype == dtype and y.shape == yr.shape
    # the residual after the mixer carries the mixer's rounding differences only
    assert normwise(to_np(r), to_np(rr)) <= (1e-5 if dtype == torch.float32 else 1e-2)
    assert_rows(to_np(y), to_np(yr), dtype, f"block ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-3, atol=1e-4)
    else:  # bf16 gates: a one-ulp input difference moves a gate by one bf16 ulp, carried by the state
        assert normwise(f.cpu().numpy(), fr.numpy()) <= TOL[dtype]


def test_tiny_lm_vs_reference_fixture():
    """configs[0]'s model: the reference's TESMLMHeadModel(TESMConfig.tiny()) from seed 0 (12 layers,
    d_model 768, vocab 151936), f32, on the reference's input ids.

    The weight scale 1/mean|w| depends on the reduction order of the mean (the device sums in float64,
    torch's CPU mean in float32), which can move a weight sitting on a rounding boundary to the next
    ternary code and so change one output column for every token.  The model therefore takes the
    oracle's codes and scales through the INT2 export loader (bit-identical to the reference's
    BitLinear quantization).  The oracle reproduces the reference's fixture exactly (CPU tests); the
    device is compared with it with its own int8 codes and ternary decisions fed in (tests/flips.py),
    per block (teacher-forced: each block fed the oracle's inputs) and end to end (every layer's mixer
    output and the logits): every row within 1e-3."""
    from oracle import int2_export
    from tesm_amd.int2 import load_int2_weights_to_model
    g, meta = load_golden("tiny_model"), golden_meta("tiny_model")
    cfg = TESMConfig.tiny()
    torch.manual_seed(meta["seed"])
    model = TESMLMHeadModel(cfg).eval()
    torch.manual_seed(meta["seed"])
    ref = ot.TESMLMHeadModel(cfg).eval()
    assert len(load_int2_weights_to_model(model, int2_export.export_model_to_int2(ref))) == 12 * 8
    ids = torch.from_numpy(g["input_ids"])
    B, L = ids.shape
    # the oracle's own run reproduces the fixture (its per-layer mixer outputs and logits)
    captured = []

    def pre(mod, args, kwargs):
        captured.append({"args": [a.clone() if torch.is_tensor(a) else a for a in args],
                         "cross": kwargs.get("cross_layer_state")})

    hooks = [blk.register_forward_pre_hook(pre, with_kwargs=True) for blk in ref.backbone.layers]
    with torch.no_grad():
        ref(ids)  # (the oracle's own logits equal the fixture's on the CPU that wrote it: CPU tests)
    for hk in hooks:
        hk.remove()
    model = model.to(DEV)
    flips = Flips(torch.float32)
    with torch.no_grad():
        # per block, teacher-forced on the oracle's inputs
        for i, (blk, c) in enumerate(zip(model.backbone.layers, captured)):
            h, r = c["args"][0], c["args"][1] if len(c["args"]) > 1 else None
            cross = c["cross"]
            mt = ModelTaps([blk], B, L)
            y, res, _ = blk(h.to(DEV), r.to(DEV) if r is not None else None,
                            cross_layer_state=cross.to(DEV) if cross is not None else None)
            mt.restore()
            rb = ref.backbone.layers[i]
            mt.install([rb], flips)
            yr, rr, _ = rb(h, r, cross_layer_state=cross)
            uninstall(rb)
            assert_rows(to_np(y), to_np(yr), torch.float32, f"block {i} ({flips.summary()})")
            assert normwise(to_np(res), to_np(rr)) <= 1e-5, i
        # end to end
        outs, routs = [], []
        hooks = [layer.mixer.register_forward_hook(lambda mod, a, out: outs.append(out[0].detach().clone()))
                 for layer in model.backbone.layers]
        mt = ModelTaps(model.backbone.layers, B, L)
        res, finals = model(ids.to(DEV))
        mt.restore()
        for hk in hooks:
            hk.remove()
        mt.install(ref.backbone.layers, flips)
        hooks = [layer.mixer.register_forward_hook(lambda mod, a, out: routs.append(out[0].detach().clone()))
                 for layer in ref.backbone.layers]
        lr, _ = ref(ids)
        for hk in hooks:
            hk.remove()
        uninstall(ref)
    assert len(outs) == 12 and len(finals) == 12 and len(routs) == 12
    for i, (o, orf) in enumerate(zip(outs, routs)):
        assert_rows(to_np(o), to_np(orf), torch.float32, f"layer {i} mixer output ({flips.summary()})")
    logits = res.logits
    assert logits.shape == (2, 16, 151936) and logits.dtype == torch.float32
    assert_rows(to_np(logits), to_np(lr), torch.float32, f"logits ({flips.summary()})")
    assert flips.code_flips <= 0.01 * flips.codes and flips.tern_flips <= 0.01 * flips.terns, flips.summary()


@pytest.mark.parametrize("mimo", [False, True])
def test_lm_prefill_and_decode_vs_oracle(mimo):
    """Prefill of 20 tokens then four one-token steps of a 2-layer model, call by call against the
    oracle with each call's decisions fed in (every block's mixer and feed-forward): every logit row
    within 1e-3."""
    cfg = _small_cfg(use_mimo=mimo, n_heads=2)
    torch.manual_seed(4)
    ref = ot.TESMLMHeadModel(cfg).eval()
    torch.manual_seed(4)
    m = TESMLMHeadModel(cfg).to(DEV).eval()
    ids = torch.randint(0, cfg.vocab_size, (3, 24), generator=torch.Generator().manual_seed(6))
    cr = {i: layer.mixer.allocate_inference_cache(3, 64) for i, layer in enumerate(ref.backbone.layers)}
    cm = m.allocate_inference_cache(3, 64)
    flips = Flips(torch.float32)

    def call(t0, t1, decode):
        mt = ModelTaps(m.backbone.layers, 3, t1 - t0, decode=decode)
        b, _ = m(ids[:, t0:t1].to(DEV), inference_params={"state_cache": cm})
        mt.restore()
        mt.install(ref.backbone.layers, flips)
        a, _ = ref(ids[:, t0:t1], inference_params={"state_cache": cr})
        uninstall(ref)
        b = b.logits if hasattr(b, "logits") else b
        return a, b

    with torch.no_grad():
        a, b = call(0, 20, False)
        assert_rows(to_np(b), to_np(a), torch.float32, f"prefill logits ({flips.summary()})")
        for t in range(20, 24):
            a, b = call(t, t + 1, True)
            assert_rows(to_np(b), to_np(a), torch.float32, f"step {t} logits ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    assert cm[0]["seq_pos"] == 24
