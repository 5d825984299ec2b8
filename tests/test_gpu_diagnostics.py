"""GPU checks of the C-ABI's diagnostics and guards: the launch log, the device status word of the
scan's bounded look-back wait, the refusal of host pointers, and the one-call BitLinear forward
whose decode-size path quantizes inside the product (bit for bit the two-launch path)."""
import ctypes

import numpy as np
import pytest
import torch

from hip_helpers import DEV, need_gpu
from tesm_amd import _lib, hip_ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def test_launch_log_names_instantiations():
    x = torch.randn(40, 300, device=DEV)
    with hip_ops.launch_log() as log:
        hip_ops.quant_act(x)
        torch.cuda.synchronize()
    assert log.kernels and all(k.startswith("quant_act_kernel<0,") for k in log.kernels), log.kernels
    with hip_ops.launch_log() as log2:
        pass
    assert log2.kernels == []                     # cleared between uses; nothing recorded when idle
    hip_ops.quant_act(x)
    with hip_ops.launch_log() as log3:
        pass
    assert log3.kernels == []                     # logging is off outside the context


def _scan_inputs(B=2, L=4096, C=128):
    g = torch.Generator().manual_seed(0)
    d = torch.sigmoid(torch.randn(B, L, C, generator=g) + 3).to(DEV)
    u = (torch.randn(B, L, C, generator=g) * 0.1).to(DEV)
    return d, u


def test_scan_give_up_sets_status_word():
    """A look-back that gives up leaves NaN states and sets bit 0 of the device status word.  The
    condition is forced from the host (a negative poll limit makes every span after the first give
    up without polling), so every wave still runs to its end."""
    d, u = _scan_inputs()
    hip_ops.device_status(clear=True)
    hip_ops.debug_scan_spin_limit(-1)
    try:
        with hip_ops.launch_log() as log:
            st, hf = hip_ops.scan(d, u, 16)
            torch.cuda.synchronize()
    finally:
        hip_ops.debug_scan_spin_limit(1 << 20)
    assert any(k.startswith("scan_lb_kernel<0,0,0,16,8,2>") for k in log.kernels), log.kernels
    assert hip_ops.device_status(clear=True) & 1
    st = st.cpu()
    span = 8 * 16                                  # eight 16-position sub-spans per workgroup
    assert torch.isfinite(st[:, :span]).all()      # the first span needs no look-back
    assert torch.isnan(st[:, span:]).all()
    assert hip_ops.device_status() == 0            # cleared
    st2, hf2 = hip_ops.scan(d, u, 16)
    torch.cuda.synchronize()
    assert hip_ops.device_status() == 0 and torch.isfinite(st2).all() and torch.isfinite(hf2).all()


def test_host_pointer_refused_before_launch():
    """A pageable host pointer is refused at the C-ABI before anything is queued (the call is also
    given an invalid layout, so nothing could launch even if the check let it through)."""
    lib = _lib.load()
    x = torch.randn(4, 64)                         # host memory
    q = torch.empty(4, 128, dtype=torch.int8, device=DEV)
    s = torch.empty(4, device=DEV)
    rs = torch.empty(4, dtype=torch.int32, device=DEV)
    rc = lib.tesm_hip_quant_act_i8(ctypes.c_void_p(x.data_ptr()), 0, 4, 64, 64, 1e-5, 7, ctypes.c_void_p(q.data_ptr()),
                                   128, ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(rs.data_ptr()), None)
    assert rc == 1
    assert b"GPU-addressable" in lib.tesm_hip_last_error()
    # device memory passes the check (and then the invalid layout is what is reported)
    xd = x.to(DEV)
    rc = lib.tesm_hip_quant_act_i8(ctypes.c_void_p(xd.data_ptr()), 0, 4, 64, 64, 1e-5, 7,
                                   ctypes.c_void_p(q.data_ptr()), 128, ctypes.c_void_p(s.data_ptr()),
                                   ctypes.c_void_p(rs.data_ptr()), None)
    assert rc == 1 and b"layout" in lib.tesm_hip_last_error()
    # pinned host memory is addressable by the GPU and accepted
    xp = x.pin_memory()
    q2, s2, _ = hip_ops.quant_act(xd)
    rc = lib.tesm_hip_quant_act_i8(ctypes.c_void_p(xp.data_ptr()), 0, 4, 64, 64, 1e-5, 1,
                                   ctypes.c_void_p(q.data_ptr()), 128, ctypes.c_void_p(s.data_ptr()),
                                   ctypes.c_void_p(rs.data_ptr()), None)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(q, q2) and torch.equal(s, s2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K", [200, 768, 1024, 1920])
@pytest.mark.parametrize("M", [5, 16, 17, 32])
@pytest.mark.parametrize("layout", ["aligned", "strided", "misaligned"])
def test_fused_quant_product_matches_two_launches(dtype, K, M, layout):
    """tesm_hip_bitlinear_fwd with fuse=1 (4 < M <= 32: the split-K product quantizes each row itself,
    skinny_fq_kernel) against fuse=0 (quant_act + the product): identical outputs, bit for bit, for
    every group count the fused kernel is instantiated for, aligned and unaligned / strided rows."""
    N = 2432
    g = torch.Generator().manual_seed(K + M)
    base = (torch.randn(M, K + 24, generator=g) * 2).to(dtype).to(DEV)
    if layout == "aligned":
        x = base[:, :K].contiguous()
    elif layout == "strided":
        x = base[:, 8:8 + K]                       # row pitch K + 24, 16-byte aligned start
    else:
        x = base[:, 1:1 + K]                       # start off the 16-byte grid
    w = torch.randn(N, K, generator=g).to(dtype).to(DEV)
    s_w, c_w = hip_ops.absmean_scale(w)
    packed = hip_ops.pack_weight(w, s_w)
    with hip_ops.launch_log() as log:
        y1 = hip_ops.bitlinear_fwd(x, packed, c_w, N, fuse=True)
        torch.cuda.synchronize()
    assert sum(k.startswith("skinny_fq_kernel<") for k in log.kernels) == 1, log.kernels
    y0 = hip_ops.bitlinear_fwd(x, packed, c_w, N, fuse=False)
    q, s, rs = hip_ops.quant_act(x)
    y2 = hip_ops.bitlinear(q, s, rs, packed, c_w, N, K, dtype)
    torch.cuda.synchronize()
    assert torch.equal(y0, y2)
    assert torch.equal(y1, y0), float((y1.float() - y0.float()).abs().max())


def test_bitlinear_module_one_call():
    """BitLinear.forward runs as one C-ABI call and matches quant_act + product."""
    from tesm_amd import BitLinear
    m = BitLinear(256, 96).to(DEV).eval()
    x = torch.randn(3, 7, 256, device=DEV)
    with torch.no_grad():
        y = m(x)
        pw = m.packed_weight()
        q, s, rs = hip_ops.quant_act(x.reshape(-1, 256))
        y2 = hip_ops.bitlinear(q, s, rs, pw.packed, pw.c_w, 96, 256, torch.float32)
    assert torch.equal(y.reshape(-1, 96), y2)
    assert np.isfinite(y.cpu().numpy()).all()


@pytest.mark.parametrize("nbytes,off", [(0, 0), (1, 0), (4095, 0), (1 << 20, 0), ((1 << 20) + 7, 3),
                                        (64 * 1024 * 1024 + 48, 0)])
def test_stream_copy(nbytes, off):
    """The streaming copy (the bandwidth reference of the measurements) copies every byte, aligned or
    not, and touches nothing past the end."""
    g = torch.Generator().manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes + off + 16,), dtype=torch.uint8, generator=g).to(DEV)
    dst = torch.zeros(nbytes + off + 16, dtype=torch.uint8, device=DEV)
    with hip_ops.launch_log() as log:
        hip_ops.stream_copy(dst[off:off + nbytes], src[off:off + nbytes])
        torch.cuda.synchronize()
    assert torch.equal(dst[off:off + nbytes], src[off:off + nbytes])
    assert not dst[:off].any() and not dst[off + nbytes:].any()
    if nbytes >= 16 and off == 0:
        assert "stream_copy_kernel" in log.kernels, log.kernels
