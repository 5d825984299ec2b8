"""CPU checks of the drop-in boundary: the C-ABI library, the host mirror of the reference API,
and the strict-backend error contract (tesm_ssm/modules/tesm.py:278-285; the reference's own
test_torch_only.py:101-104 expects RuntimeError matching "kernel_backend")."""
import os
import re

import pytest
import torch

from conftest import ROOT
from oracle import tesm_torch as ot
from tesm_amd import BitLinear, TESM, TESM_SISO, _lib


def _declared_functions():
    with open(os.path.join(ROOT, "include", "tesm_hip.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tesm_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"libtesm_hip.so does not export {name}"
    assert sorted(_lib.exported_symbols()) == declared
    assert lib.tesm_hip_abi_version() == _lib.ABI_VERSION
    assert lib.tesm_hip_kpad(1) == 128 and lib.tesm_hip_kpad(768) == 768 and lib.tesm_hip_kpad(769) == 896


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setenv("TESM_HIP_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.HipBackendUnavailable, match="not found"):
        _lib.load()


def _c_struct_fields(header_text, name):
    body = re.search(r"typedef struct " + name + r" \{(.*?)\} " + name + ";", header_text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split(None, 1)[1] if not decl.startswith("const ") else decl.split(None, 2)[2]
        for nm in names.split(","):
            fields.append(nm.strip().lstrip("*").strip())
    return fields


def test_struct_layout_matches_header(tmp_path):
    """Every ctypes descriptor has the C struct's field names, offsets and size (compiled with gcc)."""
    import ctypes
    import subprocess
    with open(os.path.join(ROOT, "include", "tesm_hip.h")) as f:
        text = f.read()
    structs = {"tesm_hip_linear": _lib.Linear, "tesm_hip_ent_quant": _lib.EntQuant,
               "tesm_hip_output_gate": _lib.OutputGate, "tesm_hip_siso_layer": _lib.SisoLayer,
               "tesm_hip_siso_step": _lib.SisoStep, "tesm_hip_mimo_layer": _lib.MimoLayer,
               "tesm_hip_mimo_step": _lib.MimoStep, "tesm_hip_rmsnorm": _lib.RmsNorm, "tesm_hip_ffn": _lib.Ffn,
               "tesm_hip_taps": _lib.Taps}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "tesm_hip.h"', "int main(void) {"]
    for cname, py in structs.items():
        fields = _c_struct_fields(text, cname)
        assert fields == [f[0] for f in py._fields_], cname
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fld in fields:
            lines.append(f'printf("{cname} {fld} %zu\\n", offsetof({cname}, {fld}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l.strip()}
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for fld, _ in py._fields_:
            assert got[(cname, fld)] == getattr(py, fld).offset, (cname, fld)


def test_seeded_construction_matches_reference_parameters():
    kw = dict(d_model=64, d_state=32, ent_rank=8, entanglement_window=8, decay_init_bias=1.0, max_seq_len=64)
    torch.manual_seed(3)
    ref = ot.TESM_SISO(**kw)
    torch.manual_seed(3)
    mine = TESM_SISO(**kw)
    rs, ms = ref.state_dict(), mine.state_dict()
    assert set(rs) == set(ms)
    for k in rs:
        assert torch.equal(rs[k], ms[k]), k
    assert TESM is TESM_SISO


def test_global_window_construction_matches_reference():
    torch.manual_seed(1)
    ref = ot.TESM_SISO(d_model=32, d_state=16, ent_rank=8, entanglement_window=0)
    torch.manual_seed(1)
    mine = TESM_SISO(d_model=32, d_state=16, ent_rank=8, entanglement_window=0)
    for k, v in ref.state_dict().items():
        assert torch.equal(v, mine.state_dict()[k]), k


def test_strict_backend_errors_on_cpu():
    bl = BitLinear(16, 4).eval()
    with torch.no_grad(), pytest.raises(RuntimeError, match="kernel_backend"):
        bl(torch.randn(2, 16))
    m = TESM_SISO(d_model=16, d_state=8, ent_rank=4, entanglement_window=4, max_seq_len=8).eval()
    with torch.no_grad(), pytest.raises(RuntimeError, match="kernel_backend"):
        m(torch.randn(1, 3, 16))
    with torch.no_grad(), pytest.raises(ValueError, match="exceeds max_seq_len"):
        m(torch.randn(1, 9, 16))
    with pytest.raises(ValueError, match="d_state must be positive"):
        TESM_SISO(d_model=16, d_state=0)


def test_empty_sequence_returns_input():
    m = TESM_SISO(d_model=16, d_state=8, ent_rank=4, entanglement_window=4, max_seq_len=8).eval()
    u = torch.randn(2, 0, 16)
    with torch.no_grad():
        out, fin = m(u)
    assert out is u and fin is None


def test_host_tensors_are_rejected_before_any_launch():
    """A CPU tensor's address must never reach a kernel (it would be dereferenced by the GPU)."""
    from tesm_amd import hip_ops
    q = torch.randn(1, 4, 8)
    with pytest.raises(RuntimeError, match="ROCm device"):
        hip_ops.local_ent(q, q, torch.zeros(4, 4, 2), torch.randn(1, 4, 16), torch.zeros(4), 4, 0.1, 0.2)
    with pytest.raises(RuntimeError, match="ROCm device"):
        hip_ops.scan(torch.rand(1, 4, 8), torch.rand(1, 4, 8))
    with pytest.raises(RuntimeError, match="ROCm device"):
        hip_ops.quant_act(torch.randn(2, 8))


def test_lm_construction_matches_reference():
    """TESMLMHeadModel(tiny()) from seed 0 holds the reference's parameters (the fingerprints the
    reference wrote: shape, first values, sum), and a small model equals the oracle's state_dict."""
    from conftest import golden_meta
    from tesm_amd import TESMConfig, TESMLMHeadModel
    meta = golden_meta("tiny_model")
    torch.manual_seed(meta["seed"])
    sd = TESMLMHeadModel(TESMConfig.tiny()).state_dict()
    for k, fp in meta["fingerprints"].items():
        if k not in sd:  # co-occurrence buffers of the reference: zero-filled, no RNG
            assert fp["abs_sum"] == 0.0, k
            continue
        v = sd[k].detach()
        assert list(v.shape) == fp["shape"], k
        assert [float(a) for a in v.flatten()[:8]] == fp["head"], k
        assert abs(float(v.double().sum()) - fp["sum"]) <= 1e-9 * max(1.0, abs(fp["abs_sum"])), k
    cfg = TESMConfig(d_model=64, n_layer=2, d_intermediate=128, vocab_size=100, max_seq_len=32, d_state=16,
                     ent_rank=8, entanglement_window=4, use_mimo=True, n_heads=2, tie_embeddings=False)
    torch.manual_seed(2)
    ref = ot.TESMLMHeadModel(cfg).state_dict()
    torch.manual_seed(2)
    mine = TESMLMHeadModel(cfg).state_dict()
    assert set(ref) == set(mine)
    assert all(torch.equal(ref[k], mine[k]) for k in ref)


@pytest.mark.parametrize("B,L,C,cs", [(4, 2048, 256, 16), (1, 5, 16, 16), (2, 129, 33, 7), (32, 64, 256, 16),
                                      (1, 32768, 8192, 16), (3, 77, 40, 64)])
def test_scan_workspace_size(B, L, C, cs):
    """Host logic only: the scan workspace holds the chunk summaries and carries (12 B per batch row,
    chunk and channel), then the look-back flags (one int per row, chunk and 64-channel group) and one
    256-byte counter line per (row, 64-channel group), each region rounded up to 256 bytes."""
    lib = _lib.load()
    cse = max(1, min(cs, L))
    T = cse if cse >= 16 else cse * (16 // cse)
    nc = -(-L // T)
    G = -(-C // 64)
    up = lambda n: -(-n // 256) * 256
    want = up(B * nc * C * 12) + up((B * nc * G + B * G * 64) * 4)
    assert int(lib.tesm_hip_scan_ws_bytes(B, L, C, cs)) == want
    assert int(lib.tesm_hip_scan_ws_bytes(B, 0, C, cs)) == 0
