"""Pin the oracle (``oracle/``) to golden vectors written from the reference.

The vectors come from ``tests/golden/gen_fixtures.py`` (reference torch path,
CPU, this container).  The oracle runs the same torch ops in the same order on
the same CPU, so parameters, stage outputs and final outputs must agree exactly.
"""
import numpy as np
import pytest
import torch

from conftest import golden_meta, load_golden
from hip_helpers import bf16_bits
from oracle import int_ref
from oracle import tesm_torch as ot
from tesm_amd.config import TESMConfig

BF16 = "torch.bfloat16"


def _t(a, dtype=None):
    t = torch.from_numpy(np.asarray(a))
    return t.to(dtype) if dtype is not None else t


def _params_match(module, g):
    sd = module.state_dict()
    for k, v in g.items():
        if not k.startswith("param/"):
            continue
        name = k[len("param/"):]
        assert name in sd, f"missing parameter {name}"
        got = sd[name].detach().float().numpy()
        assert got.shape == v.shape, name
        assert np.array_equal(got, v), f"parameter {name} differs (construction order / RNG)"


def _exact(a, b, what):
    if torch.is_tensor(a):
        a = a.detach()
        a = (a.float() if a.dtype == torch.bfloat16 else a).numpy()
    a = np.asarray(a)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert np.array_equal(a, b), f"{what}: max abs diff {np.max(np.abs(a - b))}"


# -- INT2 packing -----------------------------------------------------------------
def test_pack_known_answer():
    """Reference docstring KAT: [-1,0,+1,0] -> 0x64 (int2_quantization.py:12-13)."""
    assert int_ref.pack_i2(np.array([[-1, 0, 1, 0]], np.int8))[0, 0] == 0x64
    g = load_golden("pack_kat")
    assert np.array_equal(int_ref.pack_i2(g["codes"].astype(np.int8)), g["packed"])
    assert np.array_equal(int_ref.unpack_i2(g["packed"], g["codes"].shape[1]), g["codes"].astype(np.int8))


# -- BitLinear --------------------------------------------------------------------
@pytest.mark.parametrize("name", ["bl_f32_small", "bl_f32_padk", "bl_f32_gemv", "bl_bf16_small", "bl_bf16_gemv"])
def test_bitlinear_fixture(name):
    g, meta = load_golden(name), golden_meta(name)
    dt = torch.bfloat16 if meta["dtype"] == BF16 else torch.float32
    M, K, N = meta["M"], meta["K"], meta["N"]
    bl = ot.BitLinear(K, N)
    with torch.no_grad():
        bl.weight.copy_(_t(g["weight"]))
    bl = bl.to(dt).eval()
    x = _t(g["x"], dt)
    with torch.no_grad():
        _exact(bl(x), g["y"], "y")
        _exact(bl.quantized_input(x), g["qinput"], "qinput")
        _exact(bl.quantized_weight(), g["qweight"], "qweight")
        s_w = bl.weight_scale()
    _exact(s_w.reshape(1), g["s_w"], "s_w")
    # C restatement of the integer work against the reference's values
    if dt == torch.bfloat16:
        xb = x.view(torch.int16).numpy().view(np.uint16)
        wb = bl.weight.detach().view(torch.int16).numpy().view(np.uint16)
        q, s = int_ref.quant_act(xb, bf16_bits=True)
        wc = int_ref.weight_codes(wb, float(g["s_w"][0]), bf16_bits=True)
    else:
        q, s = int_ref.quant_act(g["x"])
        wc = int_ref.weight_codes(g["weight"], float(g["s_w"][0]))
    assert np.array_equal(q, g["x_codes"])
    assert np.array_equal(s, g["s_x"])
    assert np.array_equal(wc, g["w_codes"])
    assert np.array_equal(int_ref.pack_i2(wc), g["packed"])
    assert np.array_equal(int_ref.unpack_i2(g["packed"], K), wc)
    # in float32 the packer's own scale (eps 1e-8) yields the same codes; in bf16 the
    # packer works on float32 copies, so a few codes near +-0.5 may differ
    if dt == torch.float32:
        assert np.array_equal(g["packed_from_weight"], g["packed"])
    # exact integer accumulators reproduce the float output up to rounding
    acc = int_ref.bitlinear_acc(q, wc)
    c_w = (torch.ones((), dtype=dt) / torch.tensor(g["s_w"][0], dtype=dt)).float().item()
    y_int = acc.astype(np.float64) / s.astype(np.float64)[:, None] * c_w
    tol = 2e-2 if dt == torch.bfloat16 else 1e-5
    err = np.max(np.abs(y_int - g["y"])) / max(np.max(np.abs(g["y"])), 1e-30)
    assert err < tol, err


# -- TESM_SISO prefill ------------------------------------------------------------------
def build_siso(meta):
    torch.manual_seed(meta["seed"])
    m = ot.TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=meta["W"],
                     entanglement_threshold=meta["thr"], entanglement_scale=meta["scale"],
                     decay_init_bias=meta["decay_bias"], max_seq_len=max(meta["L"], 64),
                     state_scan_chunk_size=meta["chunk"], entanglement_block_size=meta["block"])
    return m.eval()


SISO_CASES = ["siso_f32", "siso_bf16", "siso_f32_cross_prev", "siso_f32_short", "siso_bf16_cross",
              "siso_f32_widerank"]


@pytest.mark.parametrize("name", SISO_CASES)
def test_siso_fixture(name):
    g, meta = load_golden(name), golden_meta(name)
    m = build_siso(meta)
    _params_match(m, g)
    dt = torch.bfloat16 if meta["dtype"] == BF16 else torch.float32
    m = m.to(dt)
    u = _t(g["u"], dt)
    cs = _t(g["cross"], dt) if "cross" in g else None
    h0 = _t(g["h0"]) if "h0" in g else None
    seen = {}
    for nm in ("in_proj", "state_proj", "ent_proj", "out_proj"):
        getattr(m, nm).register_forward_hook(lambda mod, a, o, nm=nm: seen.__setitem__(nm, o))
    with torch.no_grad():
        y, fin = m(u, cross_layer_state=cs, prev_state=h0)
        for nm in seen:
            _exact(seen[nm], g[f"{nm}/y"], nm)
        # stage calls on the reference's own stage inputs
        states = m._parallel_state_scan(_t(g["_parallel_state_scan/arg0#0"], dt),
                                        _t(g["_parallel_state_scan/arg1#0"], dt), prev_state=h0)
        _exact(states, g["_parallel_state_scan/out#0"], "scan")
        avg = m._compute_entanglement(_t(g["_compute_entanglement/arg0#0"], dt),
                                      _t(g["_compute_entanglement/arg1#0"], dt),
                                      _t(g["_compute_entanglement/arg2#0"], dt))
        _exact(avg, g["_compute_entanglement/out#0"], "entanglement")
    _exact(y, g["y"], "y")
    _exact(fin, g["final_state"], "final_state")
    _exact(m.last_entanglement_map, g["last_map"], "ternary map")


def test_siso_global_fixture():
    g, meta = load_golden("siso_global_f32"), golden_meta("siso_global_f32")
    torch.manual_seed(meta["seed"])
    m = ot.TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=0,
                     entanglement_threshold=0.08, max_seq_len=64).eval()
    _params_match(m, g)
    with torch.no_grad():
        y, fin = m(_t(g["u"]))
    _exact(y, g["y"], "y")
    _exact(fin, g["final_state"], "final_state")


# -- decode ----------------------------------------------------------------------------
DECODE_CASES = ["decode_f32_prefill", "decode_f32_empty", "decode_f32_short_prefill", "decode_f32_cross"]


def run_decode(meta, g, dt, amend=True):
    torch.manual_seed(meta["seed"])
    m = ot.TESM_SISO(d_model=meta["dm"], d_state=meta["D"], ent_rank=meta["R"], entanglement_window=meta["W"],
                     entanglement_threshold=0.08, decay_init_bias=1.0, max_seq_len=64, amend_bf16=amend).eval()
    _params_match(m, g)
    m = m.to(dt)
    u = _t(g["u"], dt)
    cs = _t(g["cross"], dt) if "cross" in g else None
    cache = m.allocate_inference_cache(meta["B"], 64)
    ip = {"state_cache": cache}
    P = meta["prefill"]
    outs = {}
    with torch.no_grad():
        if P:
            outs["prefill_y"] = m(u[:, :P], inference_params=ip, cross_layer_state=cs[:, :P] if cs is not None else None)[0]
        for s in range(meta["steps"]):
            t = P + s
            y, st = m(u[:, t:t + 1], inference_params=ip, cross_layer_state=cs[:, t] if cs is not None else None)
            outs[f"step{s}_y"], outs[f"step{s}_state"] = y, st
            outs[f"step{s}_kcache"] = cache["ent_k_cache"].clone()
            outs[f"step{s}_vcache"] = cache["ent_v_cache"].clone()
            outs[f"step{s}_cache_idx"] = np.array(cache["cache_idx"])
    return outs


@pytest.mark.parametrize("name", DECODE_CASES)
def test_decode_fixture(name):
    g, meta = load_golden(name), golden_meta(name)
    outs = run_decode(meta, g, torch.float32)
    for k, v in outs.items():
        _exact(v, g[k], k)


def test_decode_bf16_reference_raises_and_amendment_runs():
    g, meta = load_golden("decode_bf16_prefill"), golden_meta("decode_bf16_prefill")
    assert "expected scalar type" in meta["error"]
    with pytest.raises(RuntimeError, match="expected scalar type"):
        run_decode(meta, g, torch.bfloat16, amend=False)
    outs = run_decode(meta, g, torch.bfloat16, amend=True)
    _exact(outs["prefill_y"], g["prefill_y"], "prefill_y")
    assert all(torch.isfinite(v).all() for k, v in outs.items() if torch.is_tensor(v))


# -- MIMO ---------------------------------------------------------------------------------
def build_mimo(meta, amend=True):
    torch.manual_seed(meta["seed"])
    m = ot.TESMMIMO_Optimized(d_model=meta["dm"], d_state=meta["D"], n_heads=meta["H"], mimo_rank=meta["Rm"],
                              ent_rank=meta["R"], entanglement_window=meta["W"],
                              entanglement_threshold=meta["thr"], entanglement_scale=0.2, max_seq_len=64,
                              decay_init_bias=meta["decay_bias"], amend_bf16=amend).eval()
    with torch.no_grad():
        gg = torch.Generator().manual_seed(meta["seed"] + 7)
        H, Rm, D, W = meta["H"], meta["Rm"], meta["D"], meta["W"]
        m.mimo_x.copy_(torch.rand(H, Rm, D, generator=gg) + 0.25)
        m.mimo_o.copy_(torch.rand(H, Rm, D, generator=gg) + 0.25)
        m.local_entanglement_bias.copy_(torch.randn(H, W, generator=gg) * 0.3)
    return m


@pytest.mark.parametrize("name", ["mimo_f32", "mimo_f32_w3"])
def test_mimo_fixture(name):
    g, meta = load_golden(name), golden_meta(name)
    m = build_mimo(meta)
    _params_match(m, g)
    with torch.no_grad():
        y, fin = m(_t(g["u"]))
        a = m._local_ent_mimo(_t(g["_compute_local_entanglement_mimo/arg0#0"]),
                              _t(g["_compute_local_entanglement_mimo/arg1#0"]),
                              _t(g["_compute_local_entanglement_mimo/arg2#0"]),
                              _t(g["_compute_local_entanglement_mimo/arg3#0"]))
    _exact(a, g["_compute_local_entanglement_mimo/out#0"], "mimo local entanglement")
    _exact(y, g["y"], "y")
    _exact(fin, g["final_state"], "final_state")


def test_mimo_bf16_reference_raises_and_amendment_runs():
    g, meta = load_golden("mimo_bf16"), golden_meta("mimo_bf16")
    assert "same dtype" in meta["error"]
    with pytest.raises(RuntimeError, match="same dtype"):
        with torch.no_grad():
            build_mimo(meta, amend=False).to(torch.bfloat16)(_t(g["u"], torch.bfloat16))
    m = build_mimo(meta).to(torch.bfloat16)
    with torch.no_grad():
        y, _ = m(_t(g["u"], torch.bfloat16))
        _exact(m.in_proj(_t(g["u"], torch.bfloat16)), g["in_proj/y"], "in_proj")
    assert torch.isfinite(y.float()).all()


def test_mimo_bf16_stage_values():
    """The reference's own bf16 MIMO stages, recorded before its raise at tesm_mimo.py:1045: the
    oracle's bf16 forward feeds the scan and the window entanglement exactly the reference's inputs
    (in_proj, split and gates, RoPE: tesm_mimo.py:940-986), in the reference's dtypes (bf16 decay,
    float32 rank update; bf16 q, k and bias against float32 states), and each stage returns exactly
    the reference's output (tesm_mimo.py:375-392, 525-588), for every rank."""
    g, meta = load_golden("mimo_bf16"), golden_meta("mimo_bf16")
    m = build_mimo(meta).to(torch.bfloat16)
    seen = {"scan": [], "ent": []}
    scan0, ent0 = m._scan_mimo, m._local_ent_mimo
    m._scan_mimo = lambda d, u: seen["scan"].append((d, u)) or scan0(d, u)
    m._local_ent_mimo = lambda q, k, v, b: seen["ent"].append((q, k, v, b)) or ent0(q, k, v, b)
    with torch.no_grad():
        m(_t(g["u"], torch.bfloat16))
    assert len(seen["scan"]) == len(seen["ent"]) == meta["Rm"]
    scan_dt = (torch.bfloat16, torch.float32)
    ent_dt = (torch.bfloat16, torch.bfloat16, torch.float32, torch.bfloat16)
    for r in range(meta["Rm"]):
        key = "_parallel_state_scan_mimo/{}#" + str(r)
        for i, (a, dt) in enumerate(zip(seen["scan"][r], scan_dt)):
            assert a.dtype == dt, (r, i, a.dtype)
            _exact(a, g[key.format(f"arg{i}")], f"scan arg{i} rank {r}")
        with torch.no_grad():
            out = scan0(*(_t(g[key.format(f"arg{i}")], dt) for i, dt in enumerate(scan_dt)))
        assert out.dtype == torch.float32
        _exact(out, g[key.format("out")], f"scan rank {r}")
        key = "_compute_local_entanglement_mimo/{}#" + str(r)
        for i, (a, dt) in enumerate(zip(seen["ent"][r], ent_dt)):
            assert a.dtype == dt, (r, i, a.dtype)
            _exact(a, g[key.format(f"arg{i}")], f"entanglement arg{i} rank {r}")
        with torch.no_grad():
            out = ent0(*(_t(g[key.format(f"arg{i}")], dt) for i, dt in enumerate(ent_dt)))
        assert out.dtype == torch.float32
        _exact(out, g[key.format("out")], f"entanglement rank {r}")


def _bf16_twins(make, seed):
    """A float32 module whose parameters are bf16 values, and its bf16 copy."""
    m32 = make(seed)
    with torch.no_grad():
        for p in m32.parameters():
            p.copy_(p.bfloat16().float())
    m16 = make(seed)
    with torch.no_grad():
        for p, p32 in zip(m16.parameters(), m32.parameters()):
            p.copy_(p32)
    return m32, m16.to(torch.bfloat16)


def test_mimo_bf16_amendment_bounded():
    """What ``amend_bf16`` adds where the reference raises (the merged float32 tanh(E) and C reach the
    bf16 state_proj / ent_proj, tesm_mimo.py:1016-1045) is one round-to-nearest cast of each value to
    bf16 -- checked exactly here -- and the amended bf16 layer stays as close to the float32 layer on
    the same bf16-representable parameters and inputs as the reference's own SISO layer, which runs in
    bf16 without amendment, stays to its float32 twin at the same widths and seeds (rel. L2 0.043 to
    0.076 between the two dtypes here).  Bound: rel. L2 <= 0.08 and <= 1.5x the largest SISO gap."""
    meta = golden_meta("mimo_bf16")

    def mimo(seed):
        return build_mimo(dict(meta, seed=seed))

    def siso(seed):
        torch.manual_seed(seed)
        return ot.TESM_SISO(d_model=meta["dm"], d_state=meta["D"] * meta["H"], ent_rank=meta["R"],
                            entanglement_window=meta["W"], entanglement_threshold=meta["thr"],
                            entanglement_scale=0.2, decay_init_bias=meta["decay_bias"], max_seq_len=64).eval()

    def rel_l2(a, b):
        a, b = a.double(), b.double()
        return float((a - b).norm() / b.norm())

    gaps = {"mimo": [], "siso": []}
    casts = []
    for seed in (2, 5, 9):
        u = torch.randn(meta["B"], meta["L"], meta["dm"], generator=torch.Generator().manual_seed(seed)).bfloat16()
        for kind, make in (("mimo", mimo), ("siso", siso)):
            m32, m16 = _bf16_twins(make, seed)
            if kind == "mimo":
                def hook(te, c, ent, states, where):
                    # te / c as the amended path passes them on: one RNE cast of the float32 values
                    assert te.dtype == c.dtype == torch.bfloat16 and ent.dtype == torch.float32
                    assert torch.equal(te, torch.tanh(ent).to(torch.bfloat16))
                    casts.append(where)
                    return te, c
                m16.mix_hook = hook
            with torch.no_grad():
                y32, _ = m32(u.float())
                y16, _ = m16(u)
            assert y16.dtype == torch.bfloat16 and torch.isfinite(y16.float()).all()
            gaps[kind].append(rel_l2(y16, y32))
    assert len(casts) == 3
    assert max(gaps["mimo"]) <= min(0.08, 1.5 * max(gaps["siso"])), gaps


def test_exact_products_vs_int_ref():
    """``BitLinear.exact_products`` (the bf16 comparison basis of the GPU parity tests) equals the exact
    int32 product of the C oracle's codes, scaled once: out = bf16(acc / s_x * fl(1/s_w)), with acc the
    brute-force integer accumulator (int_ref.c), s_x the C oracle's per-token scale and fl(1/s_w) the
    bf16 dequantized weight magnitude (tesm.py:211-215)."""
    for M, K, N, seed in ((3, 64, 40, 0), (17, 700, 96, 1), (5, 4096, 64, 2)):
        gen = torch.Generator().manual_seed(seed)
        bl = ot.BitLinear(K, N).to(torch.bfloat16)
        with torch.no_grad():
            bl.weight.copy_(torch.randn(N, K, generator=gen).bfloat16())
        x = (torch.randn(M, K, generator=gen) * 3).bfloat16()
        x[0, :] = 0  # an all-zero row: eps-clamped scale, zero codes
        bl.exact_products = True
        with torch.no_grad():
            y = bl(x)
            s_w = bl.weight_scale()
            cw = bl.quantized_weight().float().abs().max()
        assert y.dtype == torch.bfloat16
        wc = int_ref.weight_codes(bf16_bits(bl.weight.detach()), float(s_w.float()), bf16_bits=True)
        q, sx = int_ref.quant_act(bf16_bits(x), bf16_bits=True)
        acc = int_ref.bitlinear_acc(q, wc).astype(np.float64)
        assert float(cw) == float((torch.ones((), dtype=torch.bfloat16) / s_w).float())
        want = torch.from_numpy(acc / sx.astype(np.float64)[:, None] * float(cw)).to(torch.bfloat16)
        _exact(y, want.float().numpy(), f"exact products M{M} K{K} N{N}")
        # and F.linear of the dequantized bf16 operands (the reference's own arithmetic) is not exact:
        # it differs from the exact product by rounding only
        bl.exact_products = False
        with torch.no_grad():
            yf = bl(x).double()
        assert float((yf - want.double()).abs().max()) <= 2 ** -6 * float(want.double().abs().max())


def test_mimo_decode_fixture():
    g, meta = load_golden("mimo_decode_f32"), golden_meta("mimo_decode_f32")
    torch.manual_seed(meta["seed"])
    m = ot.TESMMIMO_Optimized(d_model=meta["dm"], d_state=meta["D"], n_heads=meta["H"], mimo_rank=meta["Rm"],
                              ent_rank=meta["R"], entanglement_window=meta["W"], entanglement_threshold=0.05,
                              max_seq_len=64).eval()
    _params_match(m, g)
    u = _t(g["u"])
    cache = m.allocate_inference_cache(meta["B"], 64)
    ip = {"state_cache": cache}
    P = meta["prefill"]
    with torch.no_grad():
        _exact(m(u[:, :P], inference_params=ip)[0], g["prefill_y"], "prefill")
        for s in range(meta["steps"]):
            y, st = m(u[:, P + s:P + s + 1], inference_params=ip)
            _exact(y, g[f"step{s}_y"], f"step{s}")
            _exact(st, g[f"step{s}_state"], f"state{s}")


# -- config presets and the tiny() LM ------------------------------------------
def test_config_presets_match_reference():
    ref = golden_meta("_config_presets")
    for name, d in ref.items():
        mine = (TESMConfig() if name == "default" else getattr(TESMConfig, name)()).to_dict()
        assert mine == d, name
    assert TESMConfig.from_dict(TESMConfig.small().to_dict()) == TESMConfig.small()


def test_tiny_model_fixture():
    g, meta = load_golden("tiny_model"), golden_meta("tiny_model")
    cfg = TESMConfig.tiny()
    torch.manual_seed(meta["seed"])
    model = ot.TESMLMHeadModel(cfg).eval()
    sd = model.state_dict()
    for k, fp in meta["fingerprints"].items():
        if k not in sd:  # co-occurrence buffers: zero-filled, consume no RNG, unused by logits
            assert k in ("related_token_strengths", "token_freq") and fp["abs_sum"] == 0.0, k
            continue
        v = sd[k].detach()
        assert list(v.shape) == fp["shape"], k
        assert [float(a) for a in v.flatten()[:8]] == fp["head"], k
        assert abs(float(v.double().sum()) - fp["sum"]) <= 1e-9 * max(1.0, abs(fp["abs_sum"])), k
    ids = _t(g["input_ids"])
    outs = []
    with torch.no_grad():
        logits, _ = model(ids, record_mixer_outputs=outs)
    for i, o in enumerate(outs):
        _exact(o, g[f"mixer{i}_y"], f"mixer{i}")
    _exact(logits[..., :64], g["logits_head"], "logits")
    assert np.array_equal(logits.argmax(-1).numpy(), g["logits_argmax"])
    np.testing.assert_allclose(logits.double().sum(-1).numpy(), g["logits_rowsum"], rtol=1e-9, atol=1e-6)
