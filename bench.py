#!/usr/bin/env python3
"""Benchmark of the TESM forward hot path on one MI355X; prints ONE JSON line.

Workload: one TESM_SISO prefill forward at base() dims with the
BASELINE overrides d_state=256, window=16 (d_model 768, ent_rank 64, thr 0.08, scale 0.2,
decay_init_bias 2.0), batch 4 x seq 2048, bf16 activations, INT2 weights, random init from
seed 0, synthetic input already resident in HBM.  A step is one layer forward (8192 tokens).

Besides the headline tokens/s the line carries:
  roofline      the dominant kernel (the in_proj int8-MFMA GEMM, M=8192 K=768 N=2432), timed
                per launch with HIP events on the stream it runs on;
  kernels       the isolated-op measurements of configs[1] and configs[2] (GEMV/GEMM, scan,
                entanglement) with rotating buffers so the 256 MB Infinity Cache cannot serve
                repeats;
  cpu_baseline  the oracle (torch restatement of the reference's torch path) timed on this
                host's cores on the same workload, bf16, repeated for about --cpu-seconds.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "TESM-layer tokens/s at base() shape; INT2 BitLinear GB/s as % of HBM peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
LAYER = dict(d_model=768, d_state=256, ent_rank=64, entanglement_window=16, entanglement_threshold=0.08,
             entanglement_scale=0.2, decay_init_bias=2.0, max_seq_len=2048, state_scan_chunk_size=16)
B, L = 4, 2048


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-kernels", action="store_true", help="skip the isolated-kernel measurements")
    p.add_argument("--no-mimo", action="store_true", help="skip the configs[4] MIMO layer measurement")
    p.add_argument("--cpu-all", action="store_true",
                   help="time every config's CPU baseline (configs[1]-[4], the MIMO layer at L 1024/2048/4096) at "
                        "the affinity core count and on one thread, print their JSON and exit (slow)")
    p.add_argument("--only", default="", help="comma list of isolated kernels to run (profiling)")
    p.add_argument("--workload", default="all",
                   choices=["all", "layer", "decode", "mimo", "global", "lm", "base", "kernels", "in_proj"],
                   help="run one measurement alone and print its JSON (for per-workload profiles)")
    p.add_argument("--mimo-reps", type=int, default=3, help="timed configs[4] forwards (profiles use more)")
    p.add_argument("--reps", type=int, default=0,
                   help="timed repetitions of a single decode / lm / base / global workload (default: its own)")
    p.add_argument("--trace-summary", metavar="CSV", default="",
                   help="summarize a rocprofv3 --kernel-trace CSV (per kernel and launch shape: calls, median, "
                        "mean, min, max microseconds) as a markdown table, then exit")
    p.add_argument("--copy-calib", action="store_true",
                   help="run one 256 MiB device-to-device copy first (a known-size reference for "
                        "FETCH_SIZE / WRITE_SIZE counter runs)")
    return p.parse_args()


def busy(torch, ms: float = 20.0):
    """Queue a spin kernel so later launches are enqueued ahead of the GPU (events then time kernels,
    not host launch latency)."""
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(int(ms * 2.0e6))


def time_back_to_back(torch, fn, n: int, warm: int = 3):
    """Average device time per launch of n back-to-back fn() launches between one event pair on the
    current stream (the launches are queued behind a device-side wait first, so host launch latency
    does not leave gaps).  The warm-up calls fn(0 .. warm - 1): with rotating buffers, warm = their
    count, so the first timed use of a buffer does not pay the library's one-time pointer check."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    busy(torch)
    e0.record()
    for i in range(n):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n * 1e-3  # seconds


def packed_codes(torch, N, ldw, device, gen):
    c = [torch.randint(0, 3, (N, ldw), dtype=torch.uint8, device=device, generator=gen) for _ in range(4)]
    return c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6)


def measure_kernels(torch, only):
    from tesm_amd import hip_ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    res = {}
    want = set(only.split(",")) if only else None

    def sel(name):
        return want is None or name in want

    # BitLinear GEMV (M=1) and GEMM (M=2048), fp32 output
    for (M, K, N) in [(1, 4096, 4096), (1, 4096, 11008), (2048, 4096, 4096)]:
        name = f"bitlinear_M{M}_K{K}_N{N}"
        if not sel(name):
            continue
        ldw = hip_ops.kpad(K) // 4
        wbytes = N * ldw
        nrot = max(1, min(128, (512 << 20) // wbytes)) if M == 1 else 1
        packs = [packed_codes(torch, N, ldw, dev, gen) for _ in range(nrot)]
        x = torch.randn(M, K, device=dev, generator=gen)
        q, s, rs = hip_ops.quant_act(x)
        c_w = torch.full((1,), 0.05, device=dev)
        out = torch.empty(M, N, device=dev)
        t = time_back_to_back(torch, lambda i: hip_ops.bitlinear(q, s, rs, packs[i % nrot], c_w, N, K, torch.float32,
                                                             out=out), 200 if M == 1 else 50, warm=max(3, nrot))
        if M == 1:
            nbytes = N * K // 4 + M * K + M * N * 4 + 8 * M + 4
            res[name] = {"us": t * 1e6, "bound": "hbm", "achieved": nbytes / t / 1e9, "unit": "GB/s",
                         "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes, "rotating_buffers": nrot}
        else:
            ops = 2 * M * N * K
            res[name] = {"us": t * 1e6, "bound": "mfma", "achieved": ops / t / 1e12, "unit": "TOP/s (int8)",
                         "frac": ops / t / 1e12 / INT8_PEAK_TOPS, "ops": ops}
        del packs
    # SISO scan + local entanglement at small() dims, W=16, B8 x L512, bf16
    Bs, Ls, D, R, W = 8, 512, 256, 48, 16
    def rotation(set_bytes):  # distinct input sets covering >= 512 MiB, past the 256 MB Infinity Cache
        return (512 << 20) // set_bytes + 1

    if sel("scan_small"):
        nrot = rotation(Bs * Ls * D * 2 * 3)  # decay, update in; states out
        sets = [(torch.sigmoid(torch.randn(Bs, Ls, D, device=dev, generator=gen)).to(torch.bfloat16),
                 torch.randn(Bs, Ls, D, device=dev, generator=gen).to(torch.bfloat16)) for _ in range(nrot)]
        t = time_back_to_back(torch, lambda i: hip_ops.scan(sets[i % nrot][0], sets[i % nrot][1], 16), 100, warm=nrot)
        nbytes = Bs * Ls * D * (2 + 2 + 2)
        res["scan_small"] = {"us": t * 1e6, "bound": "hbm", "achieved": nbytes / t / 1e9, "unit": "GB/s",
                             "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes, "rotating_buffers": nrot}
        del sets
    if sel("local_ent_small"):
        nrot = rotation(Bs * Ls * (2 * R + 2 * D) * 2)  # q, k, states in; window average out
        rope = hip_ops.rope_table(Ls, R, torch.bfloat16, dev)
        bias = torch.randn(W, device=dev, generator=gen) * 0.3
        sets = [(torch.randn(Bs, Ls, R, device=dev, generator=gen).to(torch.bfloat16),
                 torch.randn(Bs, Ls, R, device=dev, generator=gen).to(torch.bfloat16),
                 torch.randn(Bs, Ls, D, device=dev, generator=gen).to(torch.bfloat16)) for _ in range(nrot)]
        bias_r = hip_ops.window_bias(bias, 1, W, torch.bfloat16, dev)  # rounded once, as a layer keeps it
        t = time_back_to_back(torch, lambda i: hip_ops.local_ent(sets[i % nrot][0], sets[i % nrot][1], rope,
                                                             sets[i % nrot][2], bias_r, W, 0.08, 0.2,
                                                             bias_rounded=True), 100, warm=nrot)
        nbytes = Bs * Ls * (2 * R + 2 * D) * 2
        res["local_ent_small"] = {"us": t * 1e6, "bound": "hbm", "achieved": nbytes / t / 1e9, "unit": "GB/s",
                                  "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes, "rotating_buffers": nrot}
        del sets
    if sel("local_ent_quant_small"):
        nrot = rotation(Bs * Ls * (2 * R * 2 + D * 2 + 2 * (D + 8)))
        rope = hip_ops.rope_table(Ls, R, torch.bfloat16, dev)
        bias = torch.randn(W, device=dev, generator=gen) * 0.3
        sets = [(torch.randn(Bs, Ls, R, device=dev, generator=gen).to(torch.bfloat16),
                 torch.randn(Bs, Ls, R, device=dev, generator=gen).to(torch.bfloat16),
                 torch.randn(Bs, Ls, D, device=dev, generator=gen).to(torch.bfloat16)) for _ in range(nrot)]
        bias_r = hip_ops.window_bias(bias, 1, W, torch.bfloat16, dev)
        t = time_back_to_back(torch, lambda i: hip_ops.local_ent_quant(sets[i % nrot][0], sets[i % nrot][1], rope,
                                                                   sets[i % nrot][2], bias_r, W, 0.08, 0.2,
                                                                   bias_rounded=True), 100, warm=nrot)
        # q, k, states in; int8 codes + scale + rowsum of tanh(E) and C out
        nbytes = Bs * Ls * (2 * R * 2 + D * 2 + 2 * (D + 8))
        res["local_ent_quant_small"] = {"us": t * 1e6, "bound": "hbm", "achieved": nbytes / t / 1e9, "unit": "GB/s",
                                        "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes,
                                        "rotating_buffers": nrot}
        del sets
    return res


def measure_decode(torch, m, steps: int = 50, d_model: int = LAYER["d_model"]):
    """Decode of layer `m` (configs[3]'s SISO layer, or the configs[4] MIMO layer): B = 32 sequences,
    caches filled by a 64-token prefill (>= W), then one-token steps; returns the per-step time (device
    events around `steps` consecutive steps)."""
    Bd, P = 32, 64
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    n = P + 3 + steps
    u = torch.randn(Bd, n, d_model, generator=g).to(torch.bfloat16).to(dev)
    cache = m.allocate_inference_cache(Bd, n)
    ip = {"state_cache": cache}
    m(u[:, :P], inference_params=ip)
    for t in range(P, P + 3):
        m(u[:, t:t + 1], inference_params=ip)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(P + 3, P + 3 + steps):
        m(u[:, t:t + 1], inference_params=ip)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    out = {"batch": Bd, "prefill": P, "ms_per_step": ms, "tokens_per_s": Bd / (ms * 1e-3),
           "note": "one decode step per sequence, host dispatch included (no graph capture)"}
    return out


MIMO = dict(d_model=4096, d_state=2048, n_heads=4, mimo_rank=4, ent_rank=256, entanglement_window=64,
            entanglement_threshold=0.05, entanglement_scale=0.2, max_seq_len=32768)


def measure_lm(torch, steps: int = 10):
    """configs[0]'s model on the GPU: TESMLMHeadModel(TESMConfig.tiny()) from seed 0 (12 layers, d_model 768,
    vocab 151936), batch 2 x 256 tokens, forward (embeddings, 12 blocks, norm, tied LM head) in float32
    (configs[0]'s dtype) and bfloat16; random input ids."""
    from tesm_amd import TESMConfig, TESMLMHeadModel

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = TESMConfig.tiny()
    model = TESMLMHeadModel(cfg).eval().to(dev)
    ids = torch.randint(0, cfg.vocab_size, (2, 256), generator=torch.Generator().manual_seed(0)).to(dev)
    out = {"workload": "TESMLMHeadModel(tiny()) forward, B2 x L256 (configs[0]), random init seed 0"}
    with torch.no_grad():
        for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            model = model.to(dt)
            for _ in range(2):
                model(ids)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                model(ids)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            out[name] = {"ms_per_forward": ms, "tokens_per_s": 512 / (ms * 1e-3)}
    del model
    torch.cuda.empty_cache()
    return out


def measure_true_base(torch, steps: int = 20):
    """The base() preset's own layer (d_state 384, window 32; BASELINE's headline overrides them to 256 / 16),
    B4 x L2048 prefill, bf16: per-forward time."""
    from tesm_amd import TESM_SISO

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = dict(LAYER, d_state=384, entanglement_window=32)
    m = TESM_SISO(**cfg).to(dev).to(torch.bfloat16).eval()
    u = torch.randn(B, L, LAYER["d_model"], generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        for _ in range(3):
            m(u)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            m(u)
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"workload": "TESM_SISO prefill at the base() preset's own d_state 384 / window 32, B4 x L2048, bf16",
            "ms_per_forward": ms, "tokens_per_s": B * L / (ms * 1e-3)}


def measure_global(torch, steps: int = 10):
    """TESM_SISO with global causal entanglement (entanglement_window = 0, the next row after the
    local-window layer) at configs[3]'s dims, B4 x L2048 prefill, bf16: per-forward time."""
    from tesm_amd import TESM_SISO

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = dict(LAYER)
    cfg["entanglement_window"] = 0
    m = TESM_SISO(**cfg, kernel_backend="hip").to(dev).to(torch.bfloat16).eval()
    B, L = 4, LAYER["max_seq_len"]
    u = torch.randn(B, L, LAYER["d_model"], generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        for _ in range(2):
            m(u)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            m(u)
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"workload": "TESM_SISO prefill with entanglement_window=0 (global causal ternary entanglement), "
                        "configs[3] dims, B4 x L2048, bf16", "ms_per_forward": ms, "tokens_per_s": B * L / (ms * 1e-3)}


def measure_in_proj(torch, m, u, n: int = 50):
    """The layer's in_proj GEMM (M=8192, K=768, N=2432, bf16 out) launched n times back to back on the
    stream it runs on, timed with one event pair: the roofline's per-launch figure."""
    from tesm_amd import hip_ops

    dev = torch.device("cuda:0")
    M, K = B * L, LAYER["d_model"]
    N = m.in_proj.out_features
    pw = m.in_proj.packed_weight()
    q, s, rs = hip_ops.quant_act(u.reshape(M, K))
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    t = time_back_to_back(torch, lambda i: hip_ops.bitlinear(q, s, rs, pw.packed, pw.c_w, N, K, torch.bfloat16,
                                                             out=out), n)
    return t, 2 * M * N * K, M * K + N * (K // 4) + 8 * M + 2 * M * N


def measure_mimo(torch, reps: int = 3):
    """one TESMMIMO_Optimized layer at large_40b() dims (d_model 4096, d_state 2048, 4 heads,
    mimo_rank 4, ent_rank 256, window 64), batch 1 x 32768-token prefill, bf16, INT2 weights."""
    from tesm_amd import TESMMIMO_Optimized

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    m = TESMMIMO_Optimized(**MIMO).to(dev).to(torch.bfloat16).eval()
    L = MIMO["max_seq_len"]
    u = torch.randn(1, L, MIMO["d_model"], generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        m(u)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            m(u)
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del u
    with torch.no_grad():
        dec = measure_decode(torch, m, steps=30, d_model=MIMO["d_model"])
    del m
    torch.cuda.empty_cache()
    return {"workload": "TESMMIMO_Optimized prefill, large_40b dims (configs[4]), B1 x L32768, bf16",
            "ms_per_forward": ms, "tokens_per_s": L / (ms * 1e-3), "reps": reps, "decode": dec}


def gemm_traffic():
    """HBM bytes per in_proj GEMM launch from the committed FETCH_SIZE / WRITE_SIZE counter runs, scaled by
    the same counters' reading for a 256 MiB copy (profiles/in_proj_gemm_traffic.json); None if absent."""
    path = os.path.join(ROOT, "profiles", "in_proj_gemm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def progress(msg: str) -> None:
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


def affinity_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def time_cpu(fn, seconds: float, min_reps: int = 1):
    """Median-free wall rate: one warm-up call, then calls until `seconds` have passed (at least
    min_reps); returns (calls, elapsed seconds)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= min_reps:
            return n, el


def cpu_baseline(torch, seconds: float):
    """The oracle's torch path (restating the reference's kernel_backend='torch') on host cores:
    configs[3]'s layer forward with as many threads as this process may run on, and a shorter
    one-thread sample."""
    from oracle import tesm_torch as ot

    cores = affinity_cores()
    torch.manual_seed(0)
    m = ot.TESM_SISO(**LAYER).eval().to(torch.bfloat16)
    u = torch.randn(B, L, LAYER["d_model"], generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    prev = torch.get_num_threads()
    try:
        with torch.no_grad():
            torch.set_num_threads(cores)
            n, el = time_cpu(lambda: m(u), seconds)
            torch.set_num_threads(1)
            n1, el1 = time_cpu(lambda: m(u), seconds / 4)
    finally:
        torch.set_num_threads(prev)
    return {"value": n * B * L / el, "unit": "tokens/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
            "sample": f"oracle TESM_SISO.forward (torch restatement of the reference torch path), bf16, "
                      f"{B}x{L} tokens, {n} forwards in {el:.1f} s on {cores} threads (the process's affinity set)",
            "one_thread": {"value": n1 * B * L / el1, "unit": "tokens/s", "cores": 1,
                           "sample": f"{n1} forwards in {el1:.1f} s on 1 thread"}}


def cpu_suite(torch, seconds: float):
    """CPU baselines of every config (the oracle's torch path on this host), at the affinity core count
    and on one thread: configs[1] BitLinear (fake-quant F.linear, cached ternary weight, fp32),
    configs[2] scan + local entanglement (bf16 and fp32), configs[3] layer forward (bf16 and fp32) and
    B32 decode step, configs[4] MIMO layer at L 1024 / 2048 / 4096 with a linear extrapolation to the
    32768-token prefill (the full length would take hours: the reference loops over ranks, positions
    and window slots in Python)."""
    import math

    from oracle import tesm_torch as ot

    cores = affinity_cores()
    out = {"cpu": cpu_model(), "cores": cores, "kind": "port", "configs": {}}
    prev = torch.get_num_threads()

    def both(fn, secs):
        res = {}
        for th in (cores, 1):
            torch.set_num_threads(th)
            n, el = time_cpu(fn, secs if th == cores else secs / 2)
            res[f"threads_{th}"] = {"s_per_call": el / n, "calls": n}
        return res

    try:
        with torch.no_grad():
            c1 = {}
            for (M, K, N) in [(1, 4096, 4096), (1, 4096, 11008), (2048, 4096, 4096)]:
                torch.manual_seed(0)
                bl = ot.BitLinear(K, N).eval()
                x = torch.randn(M, K, generator=torch.Generator().manual_seed(0))
                r = both(lambda: bl(x), seconds)
                nbytes = N * K // 4 + M * K + M * N * 4
                for v in r.values():
                    if M == 1:
                        v["GB_per_s_of_int2_bytes"] = nbytes / v["s_per_call"] / 1e9
                    else:
                        v["TOP_per_s"] = 2 * M * N * K / v["s_per_call"] / 1e12
                c1[f"M{M}_K{K}_N{N}"] = r
                progress(f"cpu configs[1] M{M} K{K} N{N} done")
            out["configs"]["1_bitlinear_fp32"] = c1
            c2 = {}
            for dt in (torch.bfloat16, torch.float32):
                g = torch.Generator().manual_seed(0)
                Bs, Ls, D, R, W = 8, 512, 256, 48, 16
                m = ot.TESM_SISO(d_model=512, d_state=D, ent_rank=R, entanglement_window=W,
                                 entanglement_threshold=0.08, entanglement_scale=0.2, max_seq_len=Ls).eval().to(dt)
                decay = torch.sigmoid(torch.randn(Bs, Ls, D, generator=g)).to(dt)
                upd = (torch.sigmoid(torch.randn(Bs, Ls, D, generator=g) / math.sqrt(512)) *
                       torch.tanh(torch.randn(Bs, Ls, D, generator=g) / math.sqrt(512))).to(dt)
                q = torch.randn(Bs, Ls, R, generator=g).to(dt)
                k = torch.randn(Bs, Ls, R, generator=g).to(dt)
                S = m._parallel_state_scan(decay, upd)
                c2[str(dt).split(".")[-1]] = {
                    "scan": both(lambda: m._parallel_state_scan(decay, upd), seconds / 2),
                    "local_entanglement": both(lambda: m._compute_local_entanglement(q, k, S), seconds / 2)}
                progress(f"cpu configs[2] {dt} done")
            out["configs"]["2_scan_local_ent_B8xL512"] = c2
            c3 = {}
            for dt in (torch.bfloat16, torch.float32):
                torch.manual_seed(0)
                m = ot.TESM_SISO(**LAYER).eval().to(dt)
                u = torch.randn(B, L, LAYER["d_model"], generator=torch.Generator().manual_seed(0)).to(dt)
                r = both(lambda: m(u), seconds)
                for v in r.values():
                    v["tokens_per_s"] = B * L / v["s_per_call"]
                c3[f"prefill_{str(dt).split('.')[-1]}"] = r
                ud = torch.randn(32, 65, LAYER["d_model"], generator=torch.Generator().manual_seed(1)).to(dt)
                cache = m.allocate_inference_cache(32, 128)
                m(ud[:, :64], inference_params={"state_cache": cache})

                def one_step():  # keeps stepping the same cache (positions past the prefill)
                    m(ud[:, 64:65], inference_params={"state_cache": cache})
                r = both(one_step, seconds / 2)
                for v in r.values():
                    v["tokens_per_s"] = 32 / v["s_per_call"]
                c3[f"decode_B32_{str(dt).split('.')[-1]}"] = r
                progress(f"cpu configs[3] {dt} done")
            out["configs"]["3_siso_layer_base_B4xL2048"] = c3
            c4 = {}
            mimo_cfg = dict(MIMO)
            for Lm in (1024, 2048, 4096):
                torch.manual_seed(0)
                m = ot.TESMMIMO_Optimized(**dict(mimo_cfg, max_seq_len=Lm)).eval().to(torch.bfloat16)
                u = torch.randn(1, Lm, MIMO["d_model"], generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
                torch.set_num_threads(cores)
                t0 = time.perf_counter()
                m(u)
                el = time.perf_counter() - t0
                c4[f"L{Lm}"] = {"threads": cores, "s_per_forward": el, "tokens_per_s": Lm / el}
                progress(f"cpu configs[4] L{Lm} done ({el:.1f} s)")
                del m
            # least-squares line t = a + b L through the three lengths, evaluated at 32768
            xs = [1024.0, 2048.0, 4096.0]
            ys = [c4[f"L{int(x)}"]["s_per_forward"] for x in xs]
            mx, my = sum(xs) / 3, sum(ys) / 3
            b = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
            a = my - b * mx
            t32 = a + b * 32768
            c4["extrapolated_L32768"] = {"s_per_forward": t32, "tokens_per_s": 32768 / t32,
                                         "note": "linear fit t = a + b*L through L 1024/2048/4096 (not measured)"}
            out["configs"]["4_mimo_large40b_bf16"] = c4
    finally:
        torch.set_num_threads(prev)
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_bandwidth(torch):
    """1 GiB device-to-device copies (read + write bytes per second, GB/s): the library's streaming copy
    kernel (16-byte nontemporal loads and stores, the measured ceiling that the HBM-bound kernels'
    fractions are also given against) and torch's copy_ for comparison."""
    from tesm_amd import hip_ops

    dev = torch.device("cuda:0")
    src = torch.empty(256 << 20, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    t = time_back_to_back(torch, lambda i: hip_ops.stream_copy(dst, src), 20)
    t_torch = time_back_to_back(torch, lambda i: dst.copy_(src), 20)
    del src, dst
    torch.cuda.empty_cache()
    return 2 * (1 << 30) / t / 1e9, 2 * (1 << 30) / t_torch / 1e9


def trace_summary(path: str) -> str:
    """Per kernel and launch shape of a rocprofv3 kernel-trace CSV: calls and the median / mean / min / max
    of end - start, in microseconds, as a markdown table sorted by total time."""
    import csv
    import statistics

    rows = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            grid = "x".join(r[k] for k in ("Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z") if r.get(k, "1") != "1") or "1"
            key = (r["Kernel_Name"], grid, r.get("Workgroup_Size_X", ""),
                   f"{r.get('VGPR_Count', '')} / {r.get('Accum_VGPR_Count', '')} / {r.get('LDS_Block_Size', '')}")
            rows.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in rows.values())
    out = ["| kernel | grid | wg | VGPR / AGPR / LDS | calls | median us | mean us | min us | max us | % of time |",
           "|---|---|---:|---|---:|---:|---:|---:|---:|---:|"]
    for (name, grid, wg, regs), d in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        short = name.replace("(anonymous namespace)::", "").replace("tesm::", "")
        short = short[5:] if short.startswith("void ") else short
        short = short.split("(")[0][:90]
        out.append(f"| `{short}` | {grid} | {wg} | {regs} | {len(d)} | {statistics.median(d):.2f} | "
                   f"{statistics.fmean(d):.2f} | {min(d):.2f} | {max(d):.2f} | {100 * sum(d) / total:.1f} |")
    return "\n".join(out)


def main():
    args = parse()
    if args.trace_summary:
        print(trace_summary(args.trace_summary))
        return
    if args.cpu_all:
        import torch

        print(json.dumps({"cpu_baselines": cpu_suite(torch, args.cpu_seconds)}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); multi-GPU sharding is "
              f"design-only", file=sys.stderr)
        sys.exit(2)
    import torch

    from tesm_amd import TESM_SISO, hip_ops

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    m = TESM_SISO(**LAYER).to(dev).to(torch.bfloat16).eval()
    u = torch.randn(B, L, LAYER["d_model"], generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)

    if args.copy_calib:  # a known-size plain copy (256 MiB read, 256 MiB written) for the counter runs
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        hip_ops.stream_copy(dst, src)
        torch.cuda.synchronize()
        del src, dst
    if args.workload != "all":
        with torch.no_grad():
            if args.workload == "layer":
                for _ in range(args.warmup):
                    m(u)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.steps):
                    m(u)
                e1.record()
                torch.cuda.synchronize()
                res = {"ms_per_forward": e0.elapsed_time(e1) / args.steps}
            elif args.workload == "decode":
                res = measure_decode(torch, m, **({"steps": args.reps} if args.reps else {}))
            elif args.workload == "mimo":
                res = measure_mimo(torch, reps=args.mimo_reps)
            elif args.workload == "in_proj":
                t, ops, nbytes = measure_in_proj(torch, m, u, n=args.steps)
                res = {"us": t * 1e6, "TOP_per_s": ops / t / 1e12, "frac_of_int8_peak": ops / t / 1e12 / INT8_PEAK_TOPS}
            elif args.workload == "global":
                res = measure_global(torch, **({"steps": args.reps} if args.reps else {}))
            elif args.workload == "base":
                res = measure_true_base(torch, **({"steps": args.reps} if args.reps else {}))
            elif args.workload == "kernels":
                res = measure_kernels(torch, args.only)
            else:
                res = measure_lm(torch, **({"steps": args.reps} if args.reps else {}))
        print(json.dumps({"workload": args.workload, "result": res}))
        return
    with torch.no_grad():
        for _ in range(args.warmup):
            m(u)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            m(u)
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        ms = e0.elapsed_time(e1) / args.steps

        # dominant kernel: the in_proj GEMM of the same layer on the same stream
        M, K = B * L, LAYER["d_model"]
        N = m.in_proj.out_features
        t_gemm, ops, _ = measure_in_proj(torch, m, u, n=100)
        decode = measure_decode(torch, m)
        mimo = None if args.no_mimo else measure_mimo(torch)
        glob = measure_global(torch)
        true_base = measure_true_base(torch)
        lm = measure_lm(torch)
        kernels = {} if args.no_kernels else measure_kernels(torch, args.only)
        if kernels:
            copy_gbs, copy_torch = copy_bandwidth(torch)
            kernels["copy_1GiB_GBps"] = copy_gbs
            kernels["copy_1GiB_GBps_torch"] = copy_torch
            for v in kernels.values():
                if isinstance(v, dict) and v.get("unit") == "GB/s":
                    v["frac_of_copy"] = v["achieved"] / copy_gbs
        if args.only:
            print(json.dumps({"kernels": kernels}))
            return

    value = B * L / (ms * 1e-3)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "wall_ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded randn input, random-init weights from seed 0)",
        "config": {"workload": "TESM_SISO prefill forward, base() dims with d_state=256 window=16 (configs[3])",
                   "batch": B, "seq_len": L, "d_model": 768, "d_state": 256, "ent_rank": 64, "window": 16,
                   "weights": "INT2 ternary", "activations": "bf16"},
        "roofline": {"kernel": "in_proj INT2xINT8 MFMA GEMM (M=8192, K=768, N=2432)", "bound": "mfma",
                     "achieved": ops / t_gemm / 1e12, "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": ops / t_gemm / 1e12 / INT8_PEAK_TOPS, "traffic": gemm_traffic(), "us": t_gemm * 1e6,
                     "algorithmic_bytes": M * K + N * (K // 4) + 8 * M + 2 * M * N,
                     "note": "int8 ops/s (TOP/s) against the 5.0 POP/s dense int8 MFMA peak; us = 100 back-to-back "
                             "launches between one event pair (rocprof medians: profiles/in_proj_gemm_isolated.md, and "
                             "inside the layer: profiles/siso_layer_kernels_base_bf16.md); traffic = HBM bytes per "
                             "launch from profiles/in_proj_gemm_traffic.json"},
        "decode": decode,
        "mimo_layer": mimo,
        "global_layer": glob,
        "layer_true_base": true_base,
        "lm_tiny": lm,
        "kernels": kernels,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
