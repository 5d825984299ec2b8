"""Flip-resolved parity (test infrastructure).

A device layer and the oracle make the same discrete decisions -- int8 activation codes and
ternary window decisions -- except where an upstream difference of a few ulps (exact integer vs
float GEMM accumulation, float32 vs float64 scan, device vs torch transcendental) moves a value
across a decision boundary.  These helpers

1. run the device layer with the decision taps on (``tesm_hip_debug_taps``), collecting its codes,
   scales and ternary decisions;
2. run the oracle with hooks (``BitLinear.code_hook``, ``TESM_SISO.tern_hook``) that replace each
   oracle decision by the device's, after checking that every decision that differs is a near-tie:
   the oracle's own pre-rounding value lies within ``near`` of the boundary between the two
   outcomes (codes: one step apart, value near the half-way point; ternary: score near +-thr);
3. count those flips, so that the comparison of the outputs can hold *every* row to the north-star
   tolerance (1e-3 float32, 2e-2 bfloat16).

In bfloat16 two more things are fed in, because bf16 rounding turns sub-ulp differences into
whole-ulp ones everywhere: the oracle evaluates BitLinear products exactly (``exact_products``: the
int32-accumulator arithmetic that the device implements and the north star prescribes, instead of
F.linear on bf16-rounded dequantized operands, which differs by about half an ulp per output), and
it takes the device's layer-dtype values at the three places where bf16 sums cancel -- the states
(checked normwise), tanh(E) and C = E - S (tesm.py:1231-1232), and the output gate
y = local + gate * sp + ep (tesm.py:1256-1260) -- each checked elementwise to within a couple of ulps of
the terms it is formed from.  Each stage is thus checked against the oracle's computation from the
device's previous stage.

A defect that changes decisions away from a boundary (a wrong index, scale or sign) fails step 2;
one that changes continuous values fails step 3 on the rows it touches.
"""
from __future__ import annotations

import numpy as np
import torch

from hip_helpers import DEV, normwise, to_np, unpermute_layout1
from tesm_amd import hip_ops

# near-tie width of a pre-rounding value v: REL * |v| + ABS.  float32: the paths' values differ by
# ~1e-6 relative upstream (a 10-100x margin); bfloat16: by one or two bf16 ulps (2^-8 relative
# each).  Codes: v = x * s on the 127-code scale; scores: q.k / sqrt(R) + bias near +-thr.
NEAR = {torch.float32: (1e-5, 2e-3), torch.bfloat16: (2.0 ** -6, 0.05)}
NEAR_SCORE = {torch.float32: (1e-5, 1e-4), torch.bfloat16: (2.0 ** -6, 4e-3)}
# relative difference allowed between the two paths' per-token scales (the row's absmax)
SCALE_REL = {torch.float32: 1e-5, torch.bfloat16: 2.0 ** -6}
TOL = {torch.float32: 1e-3, torch.bfloat16: 2e-2}
# bfloat16 without anything fed in: an end-to-end bound on how far the device's output drifts from the
# oracle's own (decisions made independently), so that a bf16 regression cannot hide behind the fed
# comparison -- rel. L2 within the north-star bf16 tolerance, the worst element within 5x it
UNFED = {"rel_l2": 2e-2, "normwise": 1e-1, "state": 2e-2}


class Taps:
    """Device buffers for the decision taps of one layer or feed-forward call (M tokens).

    K widths: u and y d_model, cs d_state (cs_rows rows), te and c k_te, h d_inter."""

    def __init__(self, M, k_te, d_model, dev, tern_shape=None, d_state=None, cs_rows=None, d_inter=None,
                 states=False, dtype=torch.float32):
        kp = hip_ops.kpad
        self.K = {"u": d_model, "y": d_model, "te": k_te, "c": k_te, "cs": d_state or 1, "h": d_inter or 1}
        rows = {"cs": cs_rows or M}
        for name, K in self.K.items():
            r = rows.get(name, M)
            setattr(self, "q_" + name, torch.zeros((r, kp(K)), dtype=torch.int8, device=dev))
            setattr(self, "s_" + name, torch.zeros((r,), dtype=torch.float32, device=dev))
        self.tern = torch.full(tern_shape, 7, dtype=torch.int8, device=dev) if tern_shape else None
        self.S = torch.full((M, k_te), float("nan"), device=dev) if states else None
        # the values state_proj / ent_proj quantize, in the layer dtype
        self.te = torch.full((M, k_te), float("nan"), device=dev).to(dtype)
        self.c = torch.full((M, k_te), float("nan"), device=dev).to(dtype)
        self.yv = torch.full((M, d_model), float("nan"), device=dev).to(dtype)

    def __enter__(self):
        bufs = {}
        for name in self.K:
            bufs["q_" + name] = getattr(self, "q_" + name)
            bufs["s_" + name] = getattr(self, "s_" + name)
        hip_ops.set_taps(tern=self.tern, S=self.S, te=self.te, c=self.c, yv=self.yv, **bufs)
        return self

    def __exit__(self, *exc):
        hip_ops.set_taps()
        torch.cuda.synchronize()
        return False

    def codes(self, name, rows=None):
        """(natural-order int8 codes (rows, K), float32 scales (rows,)) on the CPU (the first ``rows``)."""
        q = getattr(self, "q_" + name)[:rows].cpu().numpy()
        return unpermute_layout1(q, self.K[name]), getattr(self, "s_" + name)[:rows].cpu()


class Flips:
    """Counts and checks the decisions fed from the device into the oracle."""

    def __init__(self, dtype):
        self.dtype = dtype
        self.code_flips = 0
        self.codes = 0
        self.tern_flips = 0
        self.terns = 0
        self.mix_fed = 0

    def _near(self, v, table=NEAR):
        rel, ab = table[self.dtype]
        return rel * v.abs() + ab

    def code_hook(self, q_dev, s_dev, name="?"):
        """A BitLinear.code_hook that substitutes the device codes (M, K) and scales (M,)."""
        def hook(x, v, codes, scale):
            qd = torch.as_tensor(q_dev).reshape(codes.shape).to(codes.dtype)
            sd = torch.as_tensor(s_dev).reshape(scale.shape).to(scale.dtype)
            rel = ((sd.double() - scale.double()).abs() / scale.double().abs()).max().item()
            assert rel <= SCALE_REL[self.dtype], f"per-token scale differs beyond a near-tie: {rel:.3g}"
            diff = qd != codes
            n = int(diff.sum())
            if n:
                # the device's code must lie within the near-tie width of the oracle's unrounded value
                # (float32: one step, and only next to a rounding boundary; bfloat16: up to the few ulps
                # by which a bf16 value may differ, so two steps at the top of the code range)
                b, vv = qd.double()[diff], v.double()[diff]
                excess = (b - vv).abs() - 0.5 - self._near(vv)
                bad = excess > 0
                i = int(excess.argmax())
                assert not bool(bad.any()), (
                    f"{name}: {int(bad.sum())} of {n} differing code(s) lie away from a rounding boundary; "
                    f"worst: device code {float(b[i]):.0f} for value {float(vv[i]):.6g}")
            self.code_flips += n
            self.codes += codes.numel()
            return qd, sd
        return hook

    def tern_hook(self, dev_tern, thr, kind):
        """An oracle tern_hook that substitutes the device's ternary decisions.

        kind "local": dev_tern (B, L, W); "decode": (B, H, W) in ring read order; "mimo":
        (B, L, H, W) with entry w deciding key t - W + 1 + w; "global": (B, L, P >= L), key j of
        query i at [b, i, j] for j <= i."""
        dt = torch.as_tensor(dev_tern).to(torch.float32)

        def hook(scores, tern, where):
            if where is None or where[0] != kind:
                return tern
            if kind == "local":
                t0, t1 = where[1], where[2]
                td = dt[:, t0:t1, :].to(tern.dtype)
                W = td.shape[-1]
                pos = torch.arange(t0, t1).unsqueeze(1) - (W - 1) + torch.arange(W).unsqueeze(0)
                valid = (pos >= 0).unsqueeze(0).expand_as(tern)
            elif kind == "decode":
                td = dt.reshape(tern.shape).to(tern.dtype)
                valid = torch.ones_like(tern, dtype=torch.bool)
            elif kind == "global":
                L = tern.shape[-1]
                td = dt[:, :L, :L].to(tern.dtype)
                valid = torch.ones(L, L, dtype=torch.bool).tril().unsqueeze(0).expand_as(tern)
            else:  # mimo
                t, w = where[1], where[2]
                td = dt[:, t, :, w].reshape(tern.shape).to(tern.dtype)
                valid = torch.ones_like(tern, dtype=torch.bool)
            diff = (td != tern) & valid
            n = int(diff.sum())
            if n:
                sc = scores.double()[diff]
                assert bool((td[diff].double() - tern[diff].double()).abs().max() == 1), "a decision jumps -1 <-> +1"
                gap = (sc.abs() - thr).abs()
                bad = gap > self._near(sc, NEAR_SCORE)
                assert not bool(bad.any()), (
                    f"{int(bad.sum())} ternary decision(s) differ away from the threshold; worst gap "
                    f"{float(gap.max()):.4g} at score {float(sc[gap.argmax()]):.6g}")
            self.tern_flips += n
            self.terns += int(valid.sum())
            return torch.where(valid, td, tern)
        return hook

    def state_hook(self, dev_states, mimo_x=None):
        """An oracle state_hook that substitutes the device's layer-dtype states (bfloat16 runs: a one-ulp
        difference of a bf16 state is amplified by the cancellation in C = E - S far beyond a rounding
        tie).  The device's states must agree with the oracle's own to the bf16 tolerance, normwise;
        MIMO: the device's rank-free float32 states S give rank r's as S * mimo_x[:, r]^2."""
        d = torch.as_tensor(dev_states)

        def hook(states, where):
            if where[0] == "mimo":
                B, L, H, D = states[0].shape
                S = d.reshape(B, L, H, D).float()
                out = []
                for r, sr in enumerate(states):
                    cand = (S * mimo_x[:, r, :].float() ** 2).to(sr.dtype)
                    err = normwise(cand.numpy(), sr.float().numpy())
                    assert err <= TOL[self.dtype], f"rank {r} states differ: {err:.3g}"
                    out.append(cand)
                return out
            dd = d.reshape(states.shape).to(states.dtype)
            err = normwise(dd.float().numpy(), states.float().numpy())
            assert err <= TOL[self.dtype], f"states differ: {err:.3g}"
            return dd
        return hook

    def mix_hook(self, te_dev, c_dev):
        """An oracle mix_hook that substitutes the device's tanh(E) and C (bfloat16 runs), each element
        within what one rounding of E (and of S, and of the value itself) can move it: |d tanh E| <=
        2 ulp(tanh E) + ulp(E); |d C| <= 2 ulp(E) + 2 ulp(S) + ulp(C) (MIMO, where C is formed in float32
        and then rounded: 2 ulp(C) + 1e-5 |E|)."""
        td = torch.as_tensor(te_dev)
        cd = torch.as_tensor(c_dev)

        def ulp(x):
            a = x.double().abs().clamp_min(2.0 ** -126)
            return torch.exp2(torch.floor(torch.log2(a)) - 7)

        def hook(te, c, ent, states, where):
            t2 = td.reshape(te.shape).to(te.dtype)
            c2 = cd.reshape(c.shape).to(c.dtype)
            e = ent.double()
            tiny = 2.0 ** -24  # values this small quantize to code 0 beside any O(1) entry of their row
            lim_t = 2 * ulp(te) + ulp(e) + tiny
            if states is not None:
                lim_c = 2 * ulp(e) + 2 * ulp(states.reshape(e.shape)) + ulp(c) + tiny
            else:
                lim_c = 2 * ulp(c) + 1e-5 * e.abs() + tiny
            dt = (t2.double() - te.double()).abs()
            dc = (c2.double() - c.double()).abs()
            assert bool((dt <= lim_t).all()), f"tanh(E) differs beyond a rounding of E: {float((dt - lim_t).max()):.3g}"
            assert bool((dc <= lim_c).all()), f"C differs beyond a rounding of E and S: {float((dc - lim_c).max()):.3g}"
            self.mix_fed += 1
            return t2, c2
        return hook

    def gate_hook(self, y_dev):
        """An oracle gate_hook that substitutes the device's output-gate values y = local + gate*sp + ep
        (bfloat16 runs: the sum can cancel), each within two ulps of each of its terms and of itself."""
        yd = torch.as_tensor(y_dev)

        def ulp(x):
            a = x.double().abs().clamp_min(2.0 ** -126)
            return torch.exp2(torch.floor(torch.log2(a)) - 7)

        def hook(y, terms, where):
            y2 = yd.reshape(y.shape).to(y.dtype)
            lim = 2 * ulp(y) + 2.0 ** -24
            for t in terms:
                lim = lim + 2 * ulp(t.reshape(y.shape))
            d = (y2.double() - y.double()).abs()
            assert bool((d <= lim).all()), f"output gate y differs beyond its terms' rounding: {float((d - lim).max()):.3g}"
            self.mix_fed += 1
            return y2
        return hook

    def summary(self):
        return (f"code flips {self.code_flips}/{self.codes}, ternary flips {self.tern_flips}/{self.terns}")


def install(ref, flips, taps, tern_kind=None, thr=None, states=None, rows=None):
    """Feed the taps' decisions into oracle layer ``ref`` (SISO or MIMO); in bfloat16 runs also the
    device's ``states`` (SISO: the layer-dtype states or decode state; MIMO: the rank-free float32
    states, or the decode state) and its tanh(E) / C.  ``rows``: only the first rows (tokens) of a
    batch-1 device run, for an oracle run on that causal prefix."""
    for mod, name in ((ref.in_proj, "u"), (ref.cross_layer_q_proj, "cs"), (ref.state_proj, "te"),
                      (ref.ent_proj, "c"), (ref.out_proj, "y")):
        mod.code_hook = flips.code_hook(*taps.codes(name, rows), name=name)
        mod.exact_products = flips.dtype == torch.bfloat16
    if tern_kind is not None:
        tern = taps.tern if rows is None else taps.tern[:, :rows]
        ref.tern_hook = flips.tern_hook(tern.cpu(), ref.entanglement_threshold if thr is None else thr, tern_kind)
    if states is not None and flips.dtype == torch.bfloat16:
        ref.state_hook = flips.state_hook(states[:rows].detach().cpu(), getattr(ref, "mimo_x", None))
    if flips.dtype == torch.bfloat16:
        ref.mix_hook = flips.mix_hook(taps.te[:rows].cpu(), taps.c[:rows].cpu())
        ref.gate_hook = flips.gate_hook(taps.yv[:rows].cpu())


def install_ffn(ffn, flips, taps):
    """Feed a feed-forward call's codes (x for gate/up, h for down_proj) into oracle FeedForward ``ffn``."""
    ffn.gate_proj.code_hook = flips.code_hook(*taps.codes("u"), name="ffn x")
    ffn.down_proj.code_hook = flips.code_hook(*taps.codes("h"), name="ffn h")
    for mod in (ffn.gate_proj, ffn.down_proj):
        mod.exact_products = flips.dtype == torch.bfloat16


def uninstall(ref):
    for m in ref.modules():
        for hook in ("code_hook", "tern_hook", "state_hook", "mix_hook", "gate_hook"):
            if hasattr(m, hook):
                setattr(m, hook, None)
        if hasattr(m, "exact_products"):
            m.exact_products = False


def row_errors(a, b, floor=0.1):
    """Per-row error max|a - b| / max(max|b_row|, floor * max|b|) over the last axis."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    a2 = a.reshape(-1, a.shape[-1])
    b2 = b.reshape(-1, b.shape[-1])
    den = np.maximum(np.abs(b2).max(axis=1), floor * np.abs(b2).max())
    return np.abs(a2 - b2).max(axis=1) / np.maximum(den, 1e-30)


def assert_rows(a, b, dtype, what=""):
    err = row_errors(a, b)
    tol = TOL[dtype]
    bad = np.flatnonzero(err > tol)
    assert bad.size == 0, f"{what}: {bad.size}/{err.size} rows over {tol} (worst {err.max():.3g} at row {err.argmax()})"
    return float(err.max())


def siso_lockstep(ref, m, u, cs, P, steps, B, dtype):
    """Prefill P tokens, then `steps` one-token steps, on the device and on the oracle call by call.
    Each oracle call takes the device call's int8 codes and ternary decisions through the oracle's
    hooks, after checking that every one it would decide otherwise is a near-tie (tests/flips.py).
    Returns (device outputs, oracle outputs, Flips)."""
    flips = Flips(dtype)
    D, dm, W = m.d_state, m.d_model, m.entanglement_window
    n = max(P + steps, 64)
    caches = [m.allocate_inference_cache(B, n), ref.allocate_inference_cache(B, n)]
    outs = [{}, {}]
    ud, csd = u.to(DEV), cs.to(DEV) if cs is not None else None
    with torch.no_grad():
        if P:
            tern = (B, P, min(W, P)) if W > 0 else (B, P, (P + 63) // 64 * 64)
            with Taps(B * P, D, dm, DEV, tern, d_state=D, dtype=dtype) as tp:
                outs[0]["prefill_y"] = m(ud[:, :P], inference_params={"state_cache": caches[0]},
                                         cross_layer_state=csd[:, :P] if cs is not None else None)[0]
            install(ref, flips, tp, "local" if W > 0 else "global", states=m._last_cross_layer_state)
            outs[1]["prefill_y"] = ref(u[:, :P], inference_params={"state_cache": caches[1]},
                                       cross_layer_state=cs[:, :P] if cs is not None else None)[0]
            uninstall(ref)
        for s in range(steps):
            t = P + s
            with Taps(B, D, dm, DEV, (B, 1, max(W, 1)), d_state=D, dtype=dtype) as tp:
                y, st = m(ud[:, t:t + 1], inference_params={"state_cache": caches[0]},
                          cross_layer_state=csd[:, t] if cs is not None else None)
            install(ref, flips, tp, "decode", states=m._last_cross_layer_state)
            yr, str_ = ref(u[:, t:t + 1], inference_params={"state_cache": caches[1]},
                           cross_layer_state=cs[:, t] if cs is not None else None)
            uninstall(ref)
            for o, yy, ss, c in ((outs[0], y, st, caches[0]), (outs[1], yr, str_, caches[1])):
                o[f"step{s}_y"] = yy.clone()
                o[f"step{s}_state"] = ss.clone()
                o[f"step{s}_kcache"] = c["ent_k_cache"].clone()
                o[f"step{s}_vcache"] = c["ent_v_cache"].clone()
                o[f"step{s}_cache_idx"] = c["cache_idx"]
                o[f"step{s}_seq_pos"] = c["seq_pos"]
    if dtype == torch.bfloat16:  # the oracle on its own, for the un-fed bound
        free, cache = {}, ref.allocate_inference_cache(B, n)
        with torch.no_grad():
            if P:
                free["prefill_y"] = ref(u[:, :P], inference_params={"state_cache": cache},
                                        cross_layer_state=cs[:, :P] if cs is not None else None)[0]
            for s in range(steps):
                t = P + s
                yr, str_ = ref(u[:, t:t + 1], inference_params={"state_cache": cache},
                               cross_layer_state=cs[:, t] if cs is not None else None)
                free[f"step{s}_y"], free[f"step{s}_state"] = yr.clone(), str_.clone()
        outs[1]["unfed"] = free
    return outs[0], outs[1], flips


def assert_unfed(y, y_ref, what, state=None, state_ref=None):
    """bfloat16: the device output against the oracle's own, nothing fed in (``UNFED``)."""
    a, b = np.asarray(to_np(y), np.float64), np.asarray(to_np(y_ref), np.float64)
    r2 = float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
    nw = normwise(a, b)
    assert r2 <= UNFED["rel_l2"] and nw <= UNFED["normwise"], f"{what} un-fed: rel. L2 {r2:.3g}, normwise {nw:.3g}"
    if state is not None:
        ns = normwise(to_np(state), to_np(state_ref))
        assert ns <= UNFED["state"], f"{what} un-fed final state: normwise {ns:.3g}"
    return r2, nw


def check_siso_steps(got, want, steps, B, dtype, flips):
    """Every row of every step's output within the north-star tolerance (decisions fed in)."""
    tol = TOL[dtype]
    if "prefill_y" in got:
        assert_rows(to_np(got["prefill_y"]), to_np(want["prefill_y"]), dtype, "prefill")
    for s in range(steps):
        assert_rows(to_np(got[f"step{s}_y"]).reshape(B, -1), to_np(want[f"step{s}_y"]).reshape(B, -1), dtype,
                    f"step {s} ({flips.summary()})")
        if dtype == torch.float32:
            np.testing.assert_allclose(got[f"step{s}_state"].cpu().numpy(), want[f"step{s}_state"].numpy(),
                                       rtol=1e-4, atol=1e-5)
        else:
            # bf16 gates: a one-ulp difference of an in_proj output moves decay / write / tanh(sv) by
            # one bf16 ulp, which the float64 state then carries; the bar is normwise
            assert normwise(got[f"step{s}_state"].cpu().numpy(), want[f"step{s}_state"].numpy()) <= tol
        assert normwise(to_np(got[f"step{s}_kcache"]), to_np(want[f"step{s}_kcache"])) <= (
            1e-5 if dtype == torch.float32 else tol)
        assert normwise(to_np(got[f"step{s}_vcache"]), to_np(want[f"step{s}_vcache"])) <= (
            1e-5 if dtype == torch.float32 else tol)
        assert got[f"step{s}_cache_idx"] == want[f"step{s}_cache_idx"]
        assert got[f"step{s}_seq_pos"] == want[f"step{s}_seq_pos"]
    # decisions fed in are rare near-ties, not a systematic disagreement
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    assert flips.tern_flips <= max(4, 0.02 * flips.terns), flips.summary()
    free = want.get("unfed")
    if free is not None:
        if "prefill_y" in got:
            assert_unfed(got["prefill_y"], free["prefill_y"], "prefill")
        for s in range(steps):
            assert_unfed(got[f"step{s}_y"], free[f"step{s}_y"], f"step {s}", got[f"step{s}_state"], free[f"step{s}_state"])


class ModelTaps:
    """Per-call taps on every block of a device model (TESMLMHeadModel / MixerModel) or on one Block:
    each mixer call and each feed-forward call runs with its own taps, and ``install`` feeds them
    into the oracle's corresponding modules.  ``decode``: the next call is a one-token step."""

    def __init__(self, blocks, B, L, decode=False):
        self.blocks = list(blocks)
        self.entries = []
        for blk in self.blocks:
            mixer, mlp = blk.mixer, blk.mlp
            H = getattr(mixer, "n_heads", 1)
            mimo = hasattr(mixer, "n_heads")
            D, W, dm = mixer.d_state, mixer.entanglement_window, mixer.d_model
            M = B * L
            if decode:
                tern = (B, H, max(W, 1))
            elif W > 0:
                tern = (B, L, H, W) if mimo else (B, L, min(W, L))
            else:
                tern = (B, L, (L + 63) // 64 * 64)
            dtype = mixer.in_proj.weight.dtype
            mt = Taps(M, H * D, dm, DEV, tern, d_state=D, cs_rows=B * H if (decode and mimo) else M,
                      states=mimo and not decode, dtype=dtype)
            ft = Taps(M, 1, dm, DEV, d_inter=mlp.down_proj.in_features, dtype=dtype)
            ent = {"mixer": mt, "ffn": ft, "mimo": mimo, "states": None,
                   "orig": (mixer.forward, mlp.forward, getattr(mlp, "forward_codes", None))}
            self.entries.append(ent)
            self._wrap(blk, ent)
        self.decode = decode

    @staticmethod
    def _wrap(blk, ent):
        mixer, mlp = blk.mixer, blk.mlp
        fwd, mfwd, mcodes = ent["orig"]

        def mixer_forward(*a, **k):
            with ent["mixer"]:
                out = fwd(*a, **k)
            ent["states"] = mixer._last_cross_layer_state
            return out

        def mlp_forward(*a, **k):
            with ent["ffn"]:
                return mfwd(*a, **k)

        mixer.forward = mixer_forward
        mlp.forward = mlp_forward
        if mcodes is not None:
            def mlp_codes(*a, **k):
                with ent["ffn"]:
                    return mcodes(*a, **k)
            mlp.forward_codes = mlp_codes

    def restore(self):
        for blk, ent in zip(self.blocks, self.entries):
            for mod, name in ((blk.mixer, "forward"), (blk.mlp, "forward"), (blk.mlp, "forward_codes")):
                mod.__dict__.pop(name, None)

    def install(self, ref_blocks, flips):
        for rb, ent in zip(ref_blocks, self.entries):
            W = rb.mixer.entanglement_window
            if self.decode:
                kind = "decode"
            elif W > 0:
                kind = "mimo" if ent["mimo"] else "local"
            else:
                kind = "global"
            states = ent["mixer"].S if ent["mimo"] and not self.decode else ent["states"]
            install(rb.mixer, flips, ent["mixer"], kind, states=states)
            install_ffn(rb.mlp, flips, ent["ffn"])


def siso_prefill_check(ref, m, u, dtype, cs=None, h0=None):
    """One TESM_SISO prefill on the device (decision taps on) and on oracle ``ref`` with the device's
    decisions fed in; every row of y within the north-star tolerance.  Returns (y, final state,
    oracle y, oracle final state)."""
    B, L, dm = u.shape
    D, W = m.d_state, m.entanglement_window
    tern = (B, L, min(W, L)) if W > 0 else (B, L, (L + 63) // 64 * 64)
    flips = Flips(dtype)
    with torch.no_grad():
        with Taps(B * L, D, dm, DEV, tern, d_state=D, dtype=dtype) as tp:
            y, f = m(u.to(DEV), cross_layer_state=cs.to(DEV) if cs is not None else None,
                     prev_state=h0.to(DEV) if h0 is not None else None)
        if dtype == torch.bfloat16:
            yr0, fr0 = ref(u, cross_layer_state=cs, prev_state=h0)
            assert_unfed(y, yr0, "prefill", f, fr0)
        install(ref, flips, tp, "local" if W > 0 else "global", states=m._last_cross_layer_state)
        yr, fr = ref(u, cross_layer_state=cs, prev_state=h0)
        uninstall(ref)
    assert_rows(to_np(y), to_np(yr), dtype, f"prefill ({flips.summary()})")
    assert flips.code_flips <= max(4, 0.01 * flips.codes), flips.summary()
    assert flips.tern_flips <= max(4, 0.01 * flips.terns), flips.summary()
    return y, f, yr, fr
