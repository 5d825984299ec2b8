"""GPU parity at the BASELINE configurations' own sizes (configs[1] to configs[4]).

Each test runs the shape bench.py measures and asserts, through the C-ABI launch log, that it
reaches the kernel instantiation the measurement times.  The bar is that of the smaller tests:
integer work bit-exact; float outputs with every row within 1e-3 (float32) / 2e-2 (bfloat16) of the
oracle once the device's int8 codes and ternary decisions are fed into it (each differing decision
checked to be a near-tie, tests/flips.py).  Where the oracle cannot run the whole workload in
seconds (configs[4] at 32768 tokens) it checks a causal prefix of the device's full-size run.
"""
import math

import numpy as np
import pytest
import torch

from flips import Flips, Taps, assert_rows, assert_unfed, check_siso_steps, install, siso_lockstep, uninstall
from hip_helpers import DEV, bf16_bits, need_gpu, normwise, to_np, unpermute_layout1
from oracle import int_ref
from oracle import tesm_torch as ot
from tesm_amd import TESMMIMO_Optimized, TESM_SISO, hip_ops

pytestmark = pytest.mark.gpu

# base() dims with BASELINE's d_state / window overrides, and the true base() preset
BASE_OVERRIDE = dict(d_model=768, d_state=256, ent_rank=64, entanglement_window=16, entanglement_threshold=0.08,
                     entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=2048, state_scan_chunk_size=16)
BASE_TRUE = dict(BASE_OVERRIDE, d_state=384, entanglement_window=32)
# TESMMIMO_Optimized at large_40b() layer dims
LARGE_40B = dict(d_model=4096, d_state=2048, n_heads=4, mimo_rank=4, ent_rank=256, entanglement_window=64,
                 entanglement_threshold=0.05, entanglement_scale=0.2, max_seq_len=32768)
DT_CODE = {torch.float32: 0, torch.bfloat16: 1}


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _has(kernels, prefix):
    return any(k.startswith(prefix) for k in kernels)


def _oracle_codes(x):
    if x.dtype == torch.bfloat16:
        return int_ref.quant_act(bf16_bits(x), bf16_bits=True)
    return int_ref.quant_act(x.numpy())


def _exact_acc(q, codes):
    """Exact int32 products of int8 codes (M, K) and ternary codes (N, K): every partial sum is an
    integer below 2^24 in magnitude (K <= 8192, |q| <= 128), so float32 GEMM is exact."""
    assert q.shape[1] * 128 < (1 << 24)
    a = torch.from_numpy(q.astype(np.float32))
    b = torch.from_numpy(codes.astype(np.float32))
    return (a @ b.T).numpy().astype(np.int64)


# ---------------------------------------------------------------------------------------------
# TESMLMHeadModel(tiny()) at its stated size, B2 x L256, float32
# ---------------------------------------------------------------------------------------------
def test_cfg0_tiny_lm_at_size():
    """configs[0] at B2 x L256: the model built from seed 0 (mixer_seq_simple.py:171-345), input ids
    uniform over the vocabulary from a seed-0 generator, float32.  512 tokens run every layer product
    on the 32x32 MFMA tiles (the fixture's 32 tokens take the split-K path).  The model takes the
    oracle's ternary codes and scales through the INT2 export loader (the weight scale's reduction
    order aside, bit-identical to the reference's quantization); every layer's mixer output and the
    logits are compared with the oracle's, the device's int8 codes and ternary decisions fed in:
    every row within 1e-3."""
    from flips import ModelTaps
    from oracle import int2_export
    from tesm_amd import TESMConfig, TESMLMHeadModel
    from tesm_amd.int2 import load_int2_weights_to_model
    cfg = TESMConfig.tiny()
    B, L = 2, 256
    torch.manual_seed(0)
    model = TESMLMHeadModel(cfg).eval()
    torch.manual_seed(0)
    ref = ot.TESMLMHeadModel(cfg).eval()
    assert len(load_int2_weights_to_model(model, int2_export.export_model_to_int2(ref))) == cfg.n_layer * 8
    model = model.to(DEV)
    ids = torch.randint(0, cfg.vocab_size, (B, L), generator=torch.Generator().manual_seed(0))
    flips = Flips(torch.float32)
    outs, routs = [], []
    with torch.no_grad():
        hooks = [layer.mixer.register_forward_hook(lambda mod, a, out: outs.append(out[0].detach().clone()))
                 for layer in model.backbone.layers]
        mt = ModelTaps(model.backbone.layers, B, L)
        with hip_ops.launch_log() as log:
            res, finals = model(ids.to(DEV))
            torch.cuda.synchronize()
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
    # the layer products at 512 rows: 64x128 MFMA tiles with two direct-to-LDS stages, f32 out
    assert _has(log.kernels, "mfma32_kernel<1,4,2,1,0,0,2>"), log.kernels
    assert not _has(log.kernels, "skinny"), log.kernels
    assert len(outs) == cfg.n_layer and len(routs) == cfg.n_layer and len(finals) == cfg.n_layer
    for i, (o, orf) in enumerate(zip(outs, routs)):
        assert_rows(to_np(o), to_np(orf), torch.float32, f"configs[0] layer {i} mixer output ({flips.summary()})")
    logits = res.logits
    assert logits.shape == (B, L, cfg.vocab_size) and logits.dtype == torch.float32
    err = assert_rows(to_np(logits), to_np(lr), torch.float32, f"configs[0] logits ({flips.summary()})")
    print(f"configs[0] B2 x L256: worst logit row error {err:.3g}; {flips.summary()}")
    assert flips.code_flips <= 0.01 * flips.codes and flips.tern_flips <= 0.01 * flips.terns, flips.summary()


# ---------------------------------------------------------------------------------------------
# isolated BitLinear INT2 op
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,K,N,kernel", [(1, 4096, 4096, "gemv_kernel<64,1,1,0,2>"),
                                          (1, 4096, 11008, "gemv_kernel<64,1,1,0,2>"),
                                          (2048, 4096, 4096, "mfma32_kernel<2,4,2,2,0,0,0>")])
def test_cfg1_bitlinear_at_size(dtype, M, K, N, kernel):
    """Weights random normal fp32 quantized to ternary with a per-tensor absmean scale and packed four
    per byte; activations random normal, int8 absmax per token; float32 output as
    bench.py measures it."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(N, K, generator=g).to(dtype)
    x = torch.randn(M, K, generator=g).to(dtype)
    s_w, c_w = hip_ops.absmean_scale(w.to(DEV))
    s = float(s_w.cpu()[0])
    ref = ot.BitLinear(K, N).to(dtype)
    with torch.no_grad():
        ref.weight.copy_(w)
        s_ref = float(ref.weight_scale().float())
    assert abs(s - s_ref) <= 2 * float(torch.finfo(dtype).eps) * abs(s_ref)   # the mean's reduction order only
    wc = int_ref.weight_codes(bf16_bits(w) if dtype == torch.bfloat16 else w.numpy(), s,
                              bf16_bits=dtype == torch.bfloat16)
    packed = hip_ops.pack_weight(w.to(DEV), s_w)
    kb = (K + 3) // 4
    assert np.array_equal(packed.cpu().numpy()[:, :kb], int_ref.pack_i2(wc))
    q, sx, rs = hip_ops.quant_act(x.to(DEV))
    q_ref, sx_ref = _oracle_codes(x)
    assert np.array_equal(unpermute_layout1(q.cpu().numpy(), K), q_ref)
    assert np.array_equal(sx.cpu().numpy(), sx_ref)
    with hip_ops.launch_log() as log:
        out = hip_ops.bitlinear(q, sx, rs, packed, c_w, N, K, torch.float32)
        torch.cuda.synchronize()
    assert _has(log.kernels, kernel), log.kernels
    _, acc = hip_ops.bitlinear(q, sx, rs, packed, c_w, N, K, torch.float32, acc_dump=True)
    acc_ref = _exact_acc(q_ref, wc)
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    y_ref = acc_ref.astype(np.float64) / sx_ref.astype(np.float64)[:, None] * float(c_w.cpu()[0])
    assert normwise(out.cpu().numpy(), y_ref) < 1e-6
    # and the reference's arithmetic, F.linear of the dequantized operands (tesm.py:273-290), given the
    # device's weight scale (a weight within an ulp of a rounding boundary would otherwise follow the
    # mean's reduction order)
    if dtype == torch.float32:
        with torch.no_grad():
            deq_w = torch.from_numpy(wc.astype(np.float32)) / torch.tensor(s, dtype=torch.float32)
            y_or = torch.nn.functional.linear(ref.quantized_input(x), deq_w)
        assert_rows(out.cpu().numpy(), y_or.numpy(), torch.float32, "configs[1] vs oracle BitLinear")


# ---------------------------------------------------------------------------------------------
# isolated SISO scan + local entanglement at small() dims
# ---------------------------------------------------------------------------------------------
def _cfg2_inputs(dtype, qk_std):
    B, L, D, R, dm = 8, 512, 256, 48, 512
    g = torch.Generator().manual_seed(0)
    decay = torch.sigmoid(torch.randn(B, L, D, generator=g)).to(dtype)
    zw = torch.randn(B, L, D, generator=g) / math.sqrt(dm)
    zv = torch.randn(B, L, D, generator=g) / math.sqrt(dm)
    update = (torch.sigmoid(zw) * torch.tanh(zv)).to(dtype)
    q = (torch.randn(B, L, R, generator=g) * qk_std).to(dtype)
    k = (torch.randn(B, L, R, generator=g) * qk_std).to(dtype)
    bias = torch.randn(16, generator=g) * 0.3
    return decay, update, q, k, bias


def _cfg2_oracle_module(dtype, bias):
    m = ot.TESM_SISO(d_model=512, d_state=256, ent_rank=48, entanglement_window=16, entanglement_threshold=0.08,
                     entanglement_scale=0.2, max_seq_len=512, state_scan_chunk_size=16).eval()
    with torch.no_grad():
        m.local_entanglement_bias.copy_(bias)
    return m.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_cfg2_scan_at_size(dtype):
    decay, update, _, _, bias = _cfg2_inputs(dtype, 1.0)
    with hip_ops.launch_log() as log:
        states, hf = hip_ops.scan(decay.to(DEV), update.to(DEV), 16)
        torch.cuda.synchronize()
    dc = DT_CODE[dtype]
    assert _has(log.kernels, f"scan_lb_kernel<{dc},{dc},0,16,4,2>"), log.kernels
    ref = _cfg2_oracle_module(dtype, bias)
    with torch.no_grad():
        sr = ref._parallel_state_scan(decay, update)
    assert_rows(to_np(states), to_np(sr), dtype, "configs[2] scan states")
    np.testing.assert_allclose(hf.cpu().numpy(), ref._last_scan_state_f64.numpy(), rtol=1e-4 if dtype ==
                               torch.float32 else 2e-2, atol=1e-5)
    assert hip_ops.device_status() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("qk_std", [1 / math.sqrt(512), 1.0])
def test_cfg2_local_ent_at_size(dtype, qk_std):
    """q, k with std 1/sqrt(d_model) and std 1 (so that all three ternary values occur);
    the window average and the fused int8 codes of tanh(E) and C, with the ternary map fed in."""
    decay, update, q, k, bias = _cfg2_inputs(dtype, qk_std)
    S, _ = hip_ops.scan(decay.to(DEV), update.to(DEV), 16)
    L, R, W, thr, scale = 512, 48, 16, 0.08, 0.2
    rope = hip_ops.rope_table(L, R, dtype, DEV)
    with hip_ops.launch_log() as log:
        out = hip_ops.local_ent(q.to(DEV), k.to(DEV), rope, S, bias, W, thr, scale, outputs=("avg",), want_tern=True)
        fz = hip_ops.local_ent_quant(q.to(DEV), k.to(DEV), rope, S, bias, W, thr, scale, want_tern=True)
        torch.cuda.synchronize()
    # both the float-output op and the quantized one run on the 32-threads-per-position kernel
    assert not _has(log.kernels, "ent_scores_kernel<") and not _has(log.kernels, "ent_mix_kernel<"), log.kernels
    assert sum(k_.startswith("ent_fused2_kernel<") for k_ in log.kernels) == 2, log.kernels
    tern = out["tern"][:, :, 0, :].cpu()
    assert torch.equal(fz["tern"].cpu(), tern)
    ref = _cfg2_oracle_module(dtype, bias)
    flips = Flips(dtype)
    Sc = S.cpu()
    with torch.no_grad():
        qr, kr = ref._apply_rope(q), ref._apply_rope(k)
        ref.tern_hook = flips.tern_hook(tern, thr, "local")
        avg_r = ref._compute_local_entanglement(qr, kr, Sc)
        ref.tern_hook = None
    assert_rows(to_np(out["avg"]), to_np(avg_r), dtype, f"configs[2] window average ({flips.summary()})")
    assert flips.tern_flips <= max(4, 0.001 * flips.terns), flips.summary()
    if qk_std == 1.0:
        assert (tern == 1).any() and (tern == -1).any() and (tern == 0).any()
    # fused codes of tanh(E) and C (tesm.py:1231-1232, 206-209) against the oracle's quantization of its own E
    e = Sc + scale * (avg_r - Sc)
    for name, xin in (("te", torch.tanh(e)), ("c", e - Sc)):
        qd, sd, _ = fz[name]
        hook = flips.code_hook(unpermute_layout1(qd.cpu().numpy(), 256), sd.cpu())
        bl = ot.BitLinear(256, 8).to(dtype)
        bl.code_hook = hook
        with torch.no_grad():
            bl.quantized_input(xin.reshape(-1, 256))
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()


# ---------------------------------------------------------------------------------------------
# the TESM_SISO layer at base() dims, B4 x L2048, and its B32 decode step
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("preset", ["override", "base"])
def test_cfg3_siso_layer_at_size(dtype, preset):
    """The whole prefill forward at B4 x L2048 against the oracle; every row of y within the
    north-star tolerance with the device's decisions fed in.  'override' is BASELINE's d_state 256 /
    window 16 (the benchmarked layer), 'base' the preset's own d_state 384 / window 32."""
    cfg = BASE_OVERRIDE if preset == "override" else BASE_TRUE
    B, L = 4, 2048
    torch.manual_seed(0)
    ref = ot.TESM_SISO(**cfg).eval().to(dtype)
    torch.manual_seed(0)
    m = TESM_SISO(**cfg).to(DEV).to(dtype).eval()
    u = torch.randn(B, L, cfg["d_model"], generator=torch.Generator().manual_seed(0)).to(dtype)
    D, W = cfg["d_state"], cfg["entanglement_window"]
    flips = Flips(dtype)
    with torch.no_grad():
        with hip_ops.launch_log() as log, Taps(B * L, D, cfg["d_model"], DEV, (B, L, W), d_state=D, dtype=dtype) as tp:
            y, f = m(u.to(DEV))
        if dtype == torch.bfloat16:  # nothing fed in: the end-to-end drift from the oracle's own output
            yr0, fr0 = ref(u)
            r2, nw = assert_unfed(y, yr0, f"configs[3] {preset}", f, fr0)
            print(f"configs[3] {preset} bf16 un-fed: rel. L2 {r2:.3g}, normwise {nw:.3g}")
        install(ref, flips, tp, "local", states=m._last_cross_layer_state)
        yr, fr = ref(u)
        uninstall(ref)
    dc = DT_CODE[dtype]
    if preset == "override":
        # the benchmarked in_proj instantiation (128x256 tiles for 2048 columns, 128x128 for the rest,
        # two direct-to-LDS stages), the out_proj one (64x128 tiles, two stages) and the single-pass
        # scan with the gates fused and eight sub-spans per workgroup
        assert _has(log.kernels, f"mfma32_split_kernel<{dc},2,0>"), log.kernels
        if dtype == torch.bfloat16:  # the output gate and out_proj in one launch (32-row tiles, K 256 / 768)
            assert _has(log.kernels, "gate32_kernel<8,3,1,8,24>"), log.kernels
            assert not _has(log.kernels, "mfma32_kernel<1,4,2,1,0,"), log.kernels
        else:
            assert _has(log.kernels, f"mfma32_kernel<1,4,2,1,0,{dc},2>"), log.kernels
    assert _has(log.kernels, f"scan_lb_kernel<{dc},{dc},1,16,8,1>"), log.kernels
    if preset == "override":  # the benchmarked instantiation: 32 threads per position
        assert _has(log.kernels, "ent_fused2_kernel<"), log.kernels
    elif dtype == torch.bfloat16:  # d_state 384 / window 32 exceeds that kernel's LDS: 16 threads per position
        assert _has(log.kernels, "ent_fused_kernel<"), log.kernels
    else:  # float32 rows of 384 channels fit neither: the window sums in registers
        assert _has(log.kernels, f"ent_reg_kernel<{dc},32,"), log.kernels
    err = assert_rows(to_np(y), to_np(yr), dtype, f"configs[3] {preset} y ({flips.summary()})")
    print(f"configs[3] {preset} {dtype}: worst row error {err:.3g}; {flips.summary()}")
    assert flips.code_flips <= 0.01 * flips.codes and flips.tern_flips <= 0.01 * flips.terns, flips.summary()
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
    else:
        assert normwise(f.cpu().numpy(), fr.numpy()) <= 2e-2
    assert hip_ops.device_status() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_cfg3_decode_b32_at_size(dtype):
    """configs[3]'s incremental decode: B = 32 sequences, caches filled by a 64-token prefill (>= W),
    then one-token steps, call by call against the oracle (decisions fed in); then the benchmarked
    step (activation quantization inside the split-K products, two fewer launches) is checked bit for
    bit against the tapped step, which quantizes in separate kernels."""
    cfg = BASE_OVERRIDE
    B, P, steps = 32, 64, 3
    torch.manual_seed(0)
    ref = ot.TESM_SISO(**cfg).eval().to(dtype)
    torch.manual_seed(0)
    m = TESM_SISO(**cfg).to(DEV).to(dtype).eval()
    u = torch.randn(B, P + steps + 1, cfg["d_model"], generator=torch.Generator().manual_seed(1)).to(dtype)
    got, want, flips = siso_lockstep(ref, m, u, None, P, steps, B, dtype)
    check_siso_steps(got, want, steps, B, dtype, flips)
    # fused step == unfused step, bit for bit, from the same cache
    cache = m.allocate_inference_cache(B, P + 2)
    with torch.no_grad():
        m(u[:, :P].to(DEV), inference_params={"state_cache": cache})
        snap = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in cache.items()}
        with hip_ops.launch_log() as log:
            y1, s1 = m(u[:, P:P + 1].to(DEV), inference_params={"state_cache": cache})
            torch.cuda.synchronize()
        c1 = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in cache.items()}
        cache.update({k: (v.clone() if torch.is_tensor(v) else v) for k, v in snap.items()})
        with Taps(B, cfg["d_state"], cfg["d_model"], DEV, (B, 1, cfg["entanglement_window"]), d_state=cfg["d_state"], dtype=dtype):
            y2, s2 = m(u[:, P:P + 1].to(DEV), inference_params={"state_cache": cache})
    assert sum(k.startswith("skinny_fq_kernel<") for k in log.kernels) == 2, log.kernels
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    for key in ("ent_k_cache", "ent_v_cache", "state"):
        assert torch.equal(c1[key], cache[key]), key


# ---------------------------------------------------------------------------------------------
# TESMMIMO_Optimized at large_40b() dims
# ---------------------------------------------------------------------------------------------
def _mimo_pair(cfg, dtype, seed=0, oracle_len=None):
    torch.manual_seed(seed)
    ref = ot.TESMMIMO_Optimized(**dict(cfg, max_seq_len=oracle_len or cfg["max_seq_len"])).eval().to(dtype)
    torch.manual_seed(seed)
    m = TESMMIMO_Optimized(**cfg).to(DEV).to(dtype).eval()
    return ref, m


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_cfg4_mimo_long_vs_oracle(dtype):
    """L = 1100 (nine look-back spans of 4 x 32 positions per chain) with window 64 (the window-64 mix
    kernel) at reduced width, the whole output against the oracle, which runs the ranks uncollapsed."""
    cfg = dict(d_model=128, d_state=64, n_heads=2, mimo_rank=4, ent_rank=16, entanglement_window=64,
               entanglement_threshold=0.05, entanglement_scale=0.2, max_seq_len=1100)
    ref, m = _mimo_pair(cfg, dtype, seed=3)
    with torch.no_grad():
        gg = torch.Generator().manual_seed(10)
        for mm in (ref, m):
            mm.mimo_x.copy_((torch.rand(mm.mimo_x.shape, generator=torch.Generator().manual_seed(11)) + 0.25))
            mm.mimo_o.copy_((torch.rand(mm.mimo_o.shape, generator=torch.Generator().manual_seed(12)) + 0.25))
    u = torch.randn(1, 1100, 128, generator=gg).to(dtype)
    H, D, W = 2, 64, 64
    flips = Flips(dtype)
    with torch.no_grad():
        with hip_ops.launch_log() as log, Taps(1100, H * D, 128, DEV, (1, 1100, H, W), states=True, dtype=dtype) as tp:
            y, f = m(u.to(DEV))
        install(ref, flips, tp, "mimo", states=tp.S)
        yr, fr = ref(u)
        uninstall(ref)
    dc = DT_CODE[dtype]
    # in_proj applies the scan's gates in its epilogue; the scan streams them (its activated-gate mode)
    assert _has(log.kernels, f"mfma32_kernel<1,4,2,1,3,{dc},2>"), log.kernels
    assert _has(log.kernels, f"scan_lb_kernel<{dc},0,2,32,4,0>"), log.kernels
    assert _has(log.kernels, f"mimo_mix_kernel<{dc},true,64>"), log.kernels
    assert _has(log.kernels, f"ent_scores_mimo_kernel<{dc}>"), log.kernels
    assert_rows(to_np(y), to_np(yr), dtype, f"configs[4]-shaped MIMO L1100 ({flips.summary()})")
    assert flips.code_flips <= 0.01 * flips.codes and flips.tern_flips <= 0.01 * flips.terns, flips.summary()
    if dtype == torch.float32:
        np.testing.assert_allclose(f.cpu().numpy(), fr.numpy(), rtol=1e-4, atol=1e-5)
    else:
        assert normwise(f.cpu().numpy(), fr.numpy()) <= 2e-2


def test_cfg4_mimo_full_size():
    """configs[4] itself: B1 x L32768 at large_40b dims, bf16.  The device runs the whole prefill (the
    benchmarked kernels, named by the launch log); the oracle, which cannot run 32768 tokens in
    seconds, runs the first 512 tokens -- by causality the same rows of the output -- with the device
    run's decisions for those rows fed in.  All rows must be finite and no scan look-back may give up."""
    dtype, Lp = torch.bfloat16, 512
    cfg = LARGE_40B
    L, H, D, W, dm = cfg["max_seq_len"], cfg["n_heads"], cfg["d_state"], cfg["entanglement_window"], cfg["d_model"]
    ref, m = _mimo_pair(cfg, dtype, oracle_len=Lp)
    u = torch.randn(1, L, dm, generator=torch.Generator().manual_seed(0)).to(dtype)
    hip_ops.device_status(clear=True)
    with torch.no_grad():
        with hip_ops.launch_log() as log, Taps(L, H * D, dm, DEV, (1, L, H, W), states=True, dtype=dtype) as tp:
            y, f = m(u.to(DEV))
    assert hip_ops.device_status() == 0
    assert torch.isfinite(y.float()).all() and torch.isfinite(f).all()
    for k in ("mfma32_kernel<2,4,2,2,3,1,2>", "mfma32_kernel<2,4,2,2,0,1,2>", "mfma32_kernel<2,4,2,2,1,1,2>",
              "scan_lb_kernel<1,0,2,32,8,0>",
              "mimo_mix_kernel<1,true,64>", "ent_scores_mimo_kernel<1>"):
        assert _has(log.kernels, k), (k, log.kernels)
    # the oracle on the causal prefix, fed the device's decisions (and, bf16, states and tanh(E) / C) for
    # those rows
    flips = Flips(dtype)
    install(ref, flips, tp, "mimo", states=tp.S, rows=Lp)
    with torch.no_grad():
        yr, _ = ref(u[:, :Lp])
    uninstall(ref)
    err = assert_rows(to_np(y[:, :Lp]), to_np(yr), dtype, f"configs[4] prefix rows ({flips.summary()})")
    print(f"configs[4] prefix: worst row error {err:.3g}; {flips.summary()}")
    assert flips.code_flips <= 0.01 * flips.codes and flips.tern_flips <= 0.01 * flips.terns, flips.summary()
    _cfg4_states_full_length(m, tp, cfg, L)


def _cfg4_states_full_length(m, tp, cfg, L):
    """The rank-free states S of 64 channels (16 per head) at all 32768 positions against a float64
    sequential recurrence on the CPU (tesm_mimo.py:375-392 with the ranks collapsed).  Its inputs are
    rebuilt from the device run's own activation codes: the exact int32 products of the tapped in_proj
    codes with those channels' ternary weight codes give the sv / decay / write columns, scaled and
    rounded to bf16 as the product's epilogue does (acc * (1 / s_x) * c_w in float32), then the gates
    in the reference's bf16 op order (tesm_mimo.py:957-975).  This covers every span of the
    look-back chains, which the prefix comparison does not reach."""
    H, D, dm = cfg["n_heads"], cfg["d_state"], cfg["d_model"]
    HD = H * D
    chans = np.array([h * D + d for h in range(H) for d in np.linspace(0, D - 1, 16).astype(int)])
    cols = np.concatenate([dm + chans, dm + HD + chans, dm + 2 * HD + chans])  # sv, decay, write
    pw = m.in_proj.packed_weight()
    wc = int_ref.unpack_i2(pw.packed[torch.from_numpy(cols).to(DEV)].cpu().numpy(), dm)
    q, sx = tp.codes("u")
    acc = _exact_acc(q, wc)                                  # (L, 192) int64, exact
    c_w = np.float32(pw.c_w.float().cpu()[0])
    inv = np.float32(1.0) / sx.numpy().astype(np.float32)
    raw = (acc.astype(np.float32) * inv[:, None]) * c_w      # float32, as the epilogue
    raw = torch.from_numpy(raw).to(torch.bfloat16)
    n = len(chans)
    sv, dec, wr = raw[:, :n], raw[:, n:2 * n], raw[:, 2 * n:]
    bias = m.decay_bias.detach().reshape(-1)[torch.from_numpy(chans).to(DEV)].cpu().to(torch.bfloat16)
    decay = torch.sigmoid(dec + bias).double().numpy()
    upd = (torch.sigmoid(wr).float() * torch.tanh(sv).float()).double().numpy()
    S = np.empty((L, n))
    h = np.zeros(n)
    for t in range(L):
        h = decay[t] * h + upd[t]
        S[t] = h
    got = tp.S[:, torch.from_numpy(chans).to(DEV)].double().cpu().numpy()
    # per channel, normwise: a one-ulp gate difference (device vs torch transcendental at a bf16
    # rounding boundary) moves a state by well under 1 %; a wrong carry moves it by its own size
    den = np.abs(S).max(axis=0)
    err = np.abs(got - S).max(axis=0) / np.maximum(den, 1e-30)
    print(f"configs[4] states over L={L}: worst channel error {err.max():.3g}")
    assert np.isfinite(got).all()
    assert err.max() <= 2e-2, (err.max(), chans[err.argmax()])
    # and position by position, past the prefix the oracle covers: every 4096-position block
    for b0 in range(0, L, 4096):
        blk = np.abs(got[b0:b0 + 4096] - S[b0:b0 + 4096]).max(axis=0) / np.maximum(
            np.abs(S[b0:b0 + 4096]).max(axis=0), 1e-30)
        assert blk.max() <= 2e-2, (b0, blk.max())
