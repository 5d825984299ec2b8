"""Write the golden vectors that pin ``oracle/tesm_torch.py`` to the reference.

Runs ONLY in the build container, where the reference checkout is mounted at
``/root/reference`` (read-only).  It imports the reference's own torch path
(``kernel_backend='torch'``, CPU), runs small seeded cases and stores inputs,
parameters, intermediate stage values and outputs as ``.npz`` files next to this
script.  Nothing at test time reads the reference; the tests only read the
``.npz`` files.

What these vectors pin that closed forms and brute force cannot (survey of the
reference's own tests: it holds no fixtures for this path):
  * construction order / RNG consumption of every module at a seed,
  * torch's reduction orders and bf16 op-by-op rounding through a whole layer,
  * the LM harness plumbing (cross-layer state, decode ring buffers).

Usage:  python tests/golden/gen_fixtures.py
"""
from __future__ import annotations

import json
import os
import sys
import traceback

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    t = t.detach()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.cpu().numpy().copy()  # copy: ring buffers are later updated in place


def _state(module):
    return {f"param/{k}": _np(v) for k, v in module.state_dict().items() if v.dtype.is_floating_point}


def _capture(mod, store, prefix):
    """Record inputs/outputs of BitLinears and of the scan / entanglement calls."""
    hooks = []
    for name in ("in_proj", "state_proj", "ent_proj", "out_proj", "cross_layer_q_proj"):
        sub = getattr(mod, name, None)
        if sub is None:
            continue

        def hook(m, args, out, name=name):
            store[f"{prefix}{name}/x"] = _np(args[0])
            store[f"{prefix}{name}/y"] = _np(out)
        hooks.append(sub.register_forward_hook(hook))
    for meth in ("_parallel_state_scan", "_compute_entanglement", "_parallel_state_scan_mimo",
                 "_compute_local_entanglement_mimo"):
        if not hasattr(mod, meth):
            continue
        orig = getattr(mod, meth)

        def wrapped(*args, _orig=orig, _meth=meth, **kw):
            out = _orig(*args, **kw)
            n = sum(1 for k in store if k.startswith(f"{prefix}{_meth}/out"))
            for i, a in enumerate(args):
                if torch.is_tensor(a):
                    store[f"{prefix}{_meth}/arg{i}#{n}"] = _np(a)
            store[f"{prefix}{_meth}/out#{n}"] = _np(out)
            return out
        setattr(mod, meth, wrapped)
    return hooks


def siso_case(name, dtype, seed=0, B=2, L=40, dm=64, D=32, R=8, W=8, thr=0.08, scale=0.2,
              decay_bias=1.0, cross=False, prev=False, chunk=16, u_std=1.0, block=256):
    from tesm_ssm.modules.tesm import TESM_SISO
    torch.manual_seed(seed)
    m = TESM_SISO(d_model=dm, d_state=D, ent_rank=R, entanglement_window=W, entanglement_threshold=thr,
                  entanglement_scale=scale, decay_init_bias=decay_bias, max_seq_len=max(L, 64),
                  kernel_backend="torch", state_scan_chunk_size=chunk, entanglement_block_size=block)
    m.eval()
    store = _state(m)
    g = torch.Generator().manual_seed(seed + 1)
    u = torch.randn(B, L, dm, generator=g) * u_std
    cs = torch.randn(B, L, D, generator=g) if cross else None
    h0 = torch.randn(B, D, generator=g, dtype=torch.float64) if prev else None
    if dtype == torch.bfloat16:
        m = m.to(torch.bfloat16)
        u = u.to(torch.bfloat16)
        cs = cs.to(torch.bfloat16) if cs is not None else None
    store["u"] = _np(u)
    if cs is not None:
        store["cross"] = _np(cs)
    if h0 is not None:
        store["h0"] = h0.numpy()
    _capture(m, store, "")
    with torch.no_grad():
        y, fin = m(u, cross_layer_state=cs, prev_state=h0)
    store["y"] = _np(y)
    store["final_state"] = fin.numpy()
    store["last_map"] = _np(m.last_entanglement_map)
    meta = dict(kind="siso", dtype=str(dtype), seed=seed, B=B, L=L, dm=dm, D=D, R=R, W=W, thr=thr, scale=scale,
                decay_bias=decay_bias, cross=cross, prev=prev, chunk=chunk, u_std=u_std, block=block)
    return name, store, meta


def siso_global_case(name, seed=0, B=2, L=24, dm=64, D=16, R=8):
    from tesm_ssm.modules.tesm import TESM_SISO
    torch.manual_seed(seed)
    m = TESM_SISO(d_model=dm, d_state=D, ent_rank=R, entanglement_window=0, entanglement_threshold=0.08,
                  max_seq_len=64, kernel_backend="torch")
    m.eval()
    store = _state(m)
    u = torch.randn(B, L, dm, generator=torch.Generator().manual_seed(seed + 1))
    store["u"] = _np(u)
    _capture(m, store, "")
    with torch.no_grad():
        y, fin = m(u)
    store["y"] = _np(y)
    store["final_state"] = fin.numpy()
    return name, store, dict(kind="siso_global", seed=seed, B=B, L=L, dm=dm, D=D, R=R)


def decode_case(name, dtype, prefill, steps, seed=0, B=3, dm=64, D=32, R=8, W=8, cross=False):
    from tesm_ssm.modules.tesm import TESM_SISO
    torch.manual_seed(seed)
    m = TESM_SISO(d_model=dm, d_state=D, ent_rank=R, entanglement_window=W, entanglement_threshold=0.08,
                  decay_init_bias=1.0, max_seq_len=64, kernel_backend="torch")
    m.eval()
    store = _state(m)
    g = torch.Generator().manual_seed(seed + 1)
    u = torch.randn(B, prefill + steps, dm, generator=g)
    cs = torch.randn(B, prefill + steps, D, generator=g) if cross else None
    if dtype == torch.bfloat16:
        m = m.to(torch.bfloat16)
        u = u.to(torch.bfloat16)
        cs = cs.to(torch.bfloat16) if cs is not None else None
    store["u"] = _np(u)
    if cs is not None:
        store["cross"] = _np(cs)
    cache = m.allocate_inference_cache(B, 64)
    ip = {"state_cache": cache}
    err = None
    with torch.no_grad():
        if prefill > 0:
            y, fin = m(u[:, :prefill], inference_params=ip,
                       cross_layer_state=cs[:, :prefill] if cs is not None else None)
            store["prefill_y"] = _np(y)
        try:
            for s in range(steps):
                t = prefill + s
                y, fin = m(u[:, t:t + 1], inference_params=ip,
                           cross_layer_state=cs[:, t] if cs is not None else None)
                store[f"step{s}_y"] = _np(y)
                store[f"step{s}_state"] = fin.numpy()
                store[f"step{s}_kcache"] = _np(cache["ent_k_cache"])
                store[f"step{s}_vcache"] = _np(cache["ent_v_cache"])
                store[f"step{s}_cache_idx"] = np.array(cache["cache_idx"])
        except Exception as e:  # the reference raises for bf16 (einsum dtype mismatch)
            err = f"{type(e).__name__}: {e}"
    meta = dict(kind="decode", dtype=str(dtype), seed=seed, B=B, dm=dm, D=D, R=R, W=W, prefill=prefill,
                steps=steps, cross=cross, error=err)
    return name, store, meta


def mimo_case(name, dtype, seed=0, B=2, L=24, dm=64, D=16, H=2, Rm=2, R=8, W=8, thr=0.05, decay_bias=3.0):
    from tesm_ssm.modules.tesm_mimo import TESMMIMO_Optimized
    torch.manual_seed(seed)
    m = TESMMIMO_Optimized(d_model=dm, d_state=D, n_heads=H, mimo_rank=Rm, ent_rank=R, entanglement_window=W,
                           entanglement_threshold=thr, entanglement_scale=0.2, max_seq_len=64,
                           kernel_backend="torch", decay_init_bias=decay_bias)
    m.eval()
    with torch.no_grad():  # non-trivial rank mixing so the collapse identity is exercised
        gg = torch.Generator().manual_seed(seed + 7)
        m.mimo_x.copy_(torch.rand(H, Rm, D, generator=gg) + 0.25)
        m.mimo_o.copy_(torch.rand(H, Rm, D, generator=gg) + 0.25)
        m.local_entanglement_bias.copy_(torch.randn(H, W, generator=gg) * 0.3)
    store = _state(m)
    u = torch.randn(B, L, dm, generator=torch.Generator().manual_seed(seed + 1))
    if dtype == torch.bfloat16:
        m = m.to(torch.bfloat16)
        u = u.to(torch.bfloat16)
    store["u"] = _np(u)
    _capture(m, store, "")
    err = None
    with torch.no_grad():
        try:
            y, fin = m(u)
            store["y"] = _np(y)
            store["final_state"] = fin.numpy()
        except Exception as e:  # bf16: F.linear dtype mismatch at state_proj
            err = f"{type(e).__name__}: {e}"
    meta = dict(kind="mimo", dtype=str(dtype), seed=seed, B=B, L=L, dm=dm, D=D, H=H, Rm=Rm, R=R, W=W, thr=thr,
                decay_bias=decay_bias, error=err)
    return name, store, meta


def mimo_decode_case(name, seed=0, B=2, dm=64, D=16, H=2, Rm=2, R=8, W=8, prefill=10, steps=3):
    from tesm_ssm.modules.tesm_mimo import TESMMIMO_Optimized
    torch.manual_seed(seed)
    m = TESMMIMO_Optimized(d_model=dm, d_state=D, n_heads=H, mimo_rank=Rm, ent_rank=R, entanglement_window=W,
                           entanglement_threshold=0.05, max_seq_len=64, kernel_backend="torch")
    m.eval()
    store = _state(m)
    u = torch.randn(B, prefill + steps, dm, generator=torch.Generator().manual_seed(seed + 1))
    store["u"] = _np(u)
    cache = m.allocate_inference_cache(B, 64)
    ip = {"state_cache": cache}
    with torch.no_grad():
        y, _ = m(u[:, :prefill], inference_params=ip)
        store["prefill_y"] = _np(y)
        for s in range(steps):
            y, st = m(u[:, prefill + s:prefill + s + 1], inference_params=ip)
            store[f"step{s}_y"] = _np(y)
            store[f"step{s}_state"] = st.numpy()
    return name, store, dict(kind="mimo_decode", seed=seed, B=B, dm=dm, D=D, H=H, Rm=Rm, R=R, W=W,
                             prefill=prefill, steps=steps)


def bitlinear_case(name, dtype, M, K, N, seed=0):
    from tesm_ssm.modules.tesm import BitLinear
    from tesm_ssm.utils.int2_quantization import pack_int2_to_uint8
    torch.manual_seed(seed)
    bl = BitLinear(K, N, kernel_backend="torch")
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        bl.weight.copy_(torch.randn(N, K, generator=g))
    x = torch.randn(M, K, generator=g)
    x[0, : min(K, 3)] = 0.0
    if M > 2:
        x[2] = 0.0  # all-zero row -> eps clamp
    if dtype == torch.bfloat16:
        bl = bl.to(torch.bfloat16)
        x = x.to(torch.bfloat16)
    bl.eval()
    store = {"x": _np(x), "weight": _np(bl.weight)}
    with torch.no_grad():
        s_w = 1.0 / bl.weight.abs().mean().clamp_min(bl.bit_eps)
        codes = (bl.weight * s_w).round().clamp(-1, 1).to(torch.int8)
        store["s_w"] = _np(s_w.reshape(1))
        store["w_codes"] = codes.numpy()
        packed, _ = pack_int2_to_uint8(codes.float())
        store["packed"] = packed.numpy()
        wf = bl.weight.detach().float()
        packed_w, s_pack = pack_int2_to_uint8(wf)  # the packer's own absmean scale (eps 1e-8)
        store["packed_from_weight"] = packed_w.numpy()
        store["s_pack"] = s_pack.reshape(1).numpy()
        store["qinput"] = _np(bl.quantized_input(x))
        store["qweight"] = _np(bl.quantized_weight())
        amax = x.abs().max(dim=-1, keepdim=True).values
        s_x = 127 / amax.clamp_min(bl.bit_eps)
        store["s_x"] = _np(s_x.reshape(-1))
        store["x_codes"] = (x * s_x).round().clamp(-128, 127).to(torch.int8).numpy()
        store["y"] = _np(bl(x))
    return name, store, dict(kind="bitlinear", dtype=str(dtype), M=M, K=K, N=N, seed=seed)


def pack_kat():
    from tesm_ssm.utils.int2_quantization import pack_int2_to_uint8, unpack_uint8_to_int2
    # the reference packer takes float weights and re-derives the ternary codes itself
    v = torch.tensor([[-1, 0, 1, 0, 1, 1, -1, -1, 0, 1]], dtype=torch.float32)
    packed, scale = pack_int2_to_uint8(v)
    unpacked = unpack_uint8_to_int2(packed, scale)
    return "pack_kat", {"codes": v.numpy(), "packed": packed.numpy(), "unpacked": unpacked.numpy(),
                        "scale": scale.reshape(1).numpy()}, dict(kind="pack_kat")


def tiny_model_case(name, B=2, L=16, seed=0):
    from tesm_ssm import TESMConfig, TESMLMHeadModel
    cfg = TESMConfig.tiny()
    cfg.kernel_backend = "torch"
    torch.manual_seed(seed)
    model = TESMLMHeadModel(cfg)
    model.eval()
    store = {}
    fp = {}
    for k, v in model.state_dict().items():
        if v.dtype.is_floating_point:
            f = v.detach().double()
            fp[k] = dict(shape=list(v.shape), sum=float(f.sum()), abs_sum=float(f.abs().sum()),
                         head=[float(a) for a in v.detach().flatten()[:8]])
    ids = torch.randint(0, cfg.vocab_size, (B, L), generator=torch.Generator().manual_seed(seed + 1))
    store["input_ids"] = ids.numpy()
    outs = []
    hooks = [layer.mixer.register_forward_hook(lambda m, a, o: outs.append(o[0].detach().clone()))
             for layer in model.backbone.layers]
    with torch.no_grad():
        res, _ = model(ids)
    for h in hooks:
        h.remove()
    logits = res.logits
    store["logits_head"] = _np(logits[..., :64])
    store["logits_rowsum"] = logits.double().sum(-1).numpy()
    store["logits_rowsq"] = (logits.double() ** 2).sum(-1).numpy()
    store["logits_argmax"] = logits.argmax(-1).numpy()
    for i, o in enumerate(outs):
        store[f"mixer{i}_y"] = _np(o)
    return name, store, dict(kind="tiny_model", B=B, L=L, seed=seed, fingerprints=fp)


def config_presets():
    from tesm_ssm import TESMConfig
    names = ["tiny", "small", "small_short", "base", "medium", "long_context", "large_40b", "large_70b",
             "large_100b", "large_200b", "large_400b"]
    out = {n: getattr(TESMConfig, n)().to_dict() for n in names}
    out["default"] = TESMConfig().to_dict()
    return out


def main():
    if not os.path.isdir(os.path.join(REF, "tesm_ssm")):
        sys.exit("reference checkout not found at /root/reference; fixtures can only be regenerated there")
    sys.path.insert(0, REF)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    cases = [
        pack_kat(),
        bitlinear_case("bl_f32_small", torch.float32, 3, 64, 40),
        bitlinear_case("bl_f32_padk", torch.float32, 5, 130, 24, seed=3),
        bitlinear_case("bl_f32_gemv", torch.float32, 1, 4096, 64, seed=1),
        bitlinear_case("bl_bf16_small", torch.bfloat16, 3, 64, 40),
        bitlinear_case("bl_bf16_gemv", torch.bfloat16, 1, 4096, 64, seed=1),
        siso_case("siso_f32", torch.float32),
        siso_case("siso_bf16", torch.bfloat16),
        siso_case("siso_f32_cross_prev", torch.float32, seed=2, cross=True, prev=True, L=37, chunk=8, block=16),
        siso_case("siso_f32_short", torch.float32, seed=4, L=5),
        siso_case("siso_bf16_cross", torch.bfloat16, seed=5, cross=True, L=33, u_std=2.0),
        siso_case("siso_f32_widerank", torch.float32, seed=6, B=1, L=48, dm=96, D=64, R=64, W=16, thr=0.05),
        siso_global_case("siso_global_f32"),
        decode_case("decode_f32_prefill", torch.float32, prefill=12, steps=4),
        decode_case("decode_f32_empty", torch.float32, prefill=0, steps=10, seed=1),
        decode_case("decode_f32_short_prefill", torch.float32, prefill=5, steps=4, seed=2),
        decode_case("decode_f32_cross", torch.float32, prefill=9, steps=3, seed=3, cross=True),
        decode_case("decode_bf16_prefill", torch.bfloat16, prefill=12, steps=2, seed=4),
        mimo_case("mimo_f32", torch.float32),
        mimo_case("mimo_f32_w3", torch.float32, seed=1, L=11, W=3, H=3, Rm=3, D=8, R=4),
        mimo_case("mimo_bf16", torch.bfloat16, seed=2),
        mimo_decode_case("mimo_decode_f32"),
        tiny_model_case("tiny_model"),
    ]
    index = {}
    for name, store, meta in cases:
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **store)
        index[name] = meta
        print(f"{name}: {len(store)} arrays" + (f"  (reference raised: {meta['error'][:80]})"
                                                 if meta.get("error") else ""))
    index["_config_presets"] = config_presets()
    index["_torch_version"] = torch.__version__
    with open(os.path.join(HERE, "index.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    try:
        main()
    except Exception:
        traceback.print_exc()
        sys.exit(1)
