"""GPU parity of the fused gate projections (omx_gdn_ab_proj, deltanet.py:240-241).

a = x W_a^T and b = x W_b^T are bf16 linear maps with fp32 accumulation.  The kernel is
checked against the fp64 product of the same bf16 inputs (one bf16 rounding of the
output: within 8e-3, max-abs-normalised), against torch's bf16 F.linear (the library
GEMMs it replaces), and through autograd against F.linear's gradients (2e-2).  Shapes
cover D not a multiple of 32, Hv not a multiple of 4 or 16, M not a multiple of 64,
and Hv up to the kernel's limit of 128.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def np_(t):
    return t.detach().float().cpu().numpy()


def inputs(M, D, Hv, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).bfloat16().cuda()
    wa = (0.05 * torch.randn(Hv, D, generator=g)).bfloat16().cuda()
    wb = (0.05 * torch.randn(Hv, D, generator=g)).bfloat16().cuda()
    return x, wa, wb


@pytest.mark.parametrize("M,D,Hv", [(16384, 2048, 32), (100, 16, 4), (1, 64, 6), (130, 96, 2),
                                    (77, 40, 20), (256, 2048, 64), (65, 1024, 128)])
def test_ab_projections_match_fp64_and_library_gemms(M, D, Hv):
    from omegalax_amd import gdn_ab_projections
    print(f"ab projections M={M} D={D} Hv={Hv}", flush=True)
    sys.stdout.flush()
    x, wa, wb = inputs(M, D, Hv, M + D + Hv)
    a, b = gdn_ab_projections(x, wa, wb)
    torch.cuda.synchronize()
    x64 = np_(x).astype(np.float64)
    for got, w in ((a, wa), (b, wb)):
        assert tuple(got.shape) == (M, Hv) and got.dtype == torch.bfloat16
        assert rel(np_(got), x64 @ np_(w).astype(np.float64).T) < 8e-3
        assert rel(np_(got), np_(torch.nn.functional.linear(x, w))) < 1e-2


def test_ab_projections_keep_leading_dims_and_backward():
    from omegalax_amd import gdn_ab_projections
    print("ab projections autograd B=2 T=50 D=96 Hv=4", flush=True)
    x, wa, wb = inputs(100, 96, 4, 7)
    x = x.reshape(2, 50, 96)
    ts = [t.clone().requires_grad_(True) for t in (x, wa, wb)]
    a, b = gdn_ab_projections(*ts)
    assert tuple(a.shape) == (2, 50, 4)
    g = torch.Generator().manual_seed(8)
    da = torch.randn(2, 50, 4, generator=g).bfloat16().cuda()
    db = torch.randn(2, 50, 4, generator=g).bfloat16().cuda()
    (a.float() * da.float()).sum().add((b.float() * db.float()).sum()).backward()
    rs = [t.clone().float().requires_grad_(True) for t in (x, wa, wb)]
    F = torch.nn.functional
    (F.linear(rs[0], rs[1]) * da.float()).sum().add((F.linear(rs[0], rs[2]) * db.float()).sum()).backward()
    for t, r in zip(ts, rs):
        assert rel(np_(t.grad), np_(r.grad)) < 2e-2


def test_ab_projections_outputs_at_two_byte_alignment():
    """a and b need only bf16 alignment: outputs that start 2 bytes into a buffer (Hv % 4 == 0,
    where aligned outputs take 8-byte stores) equal the aligned call bit for bit, and the
    element before each output is left untouched."""
    from omegalax_amd import _lib, gdn_ab_projections
    from omegalax_amd.deltanet import _ptr, _stream
    M, D, Hv = 130, 96, 8
    print(f"ab projections misaligned outputs M={M} D={D} Hv={Hv}", flush=True)
    sys.stdout.flush()
    x, wa, wb = inputs(M, D, Hv, 11)
    a_ref, b_ref = gdn_ab_projections(x, wa, wb)
    bufs = [torch.full((M * Hv + 1,), 7.0, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    a, b = (t[1:].view(M, Hv) for t in bufs)
    assert _ptr(a) % 8 == 2 and _ptr(b) % 8 == 2
    _lib.call("omx_gdn_ab_proj", _ptr(x), _ptr(wa), _ptr(wb), _ptr(a), _ptr(b), M, D, Hv,
              _stream(x.device))
    torch.cuda.synchronize()
    assert torch.equal(a, a_ref) and torch.equal(b, b_ref)
    assert all(float(t[0]) == 7.0 for t in bufs)


def test_ab_projections_take_a_misaligned_hidden_view():
    """A bf16 hidden view whose storage offset is not a multiple of 8 elements (not 16-byte
    aligned) is copied to an aligned tensor first: the result equals the aligned call bit
    for bit, as does the layer's projection step that calls it."""
    from omegalax_amd import gdn_ab_projections
    from omegalax_amd.deltanet import _ptr
    M, D, Hv = 64, 2048, 32
    print(f"ab projections misaligned input view M={M} D={D} Hv={Hv}", flush=True)
    sys.stdout.flush()
    x, wa, wb = inputs(M, D, Hv, 13)
    buf = torch.empty(M * D + 1, dtype=torch.bfloat16, device="cuda")
    xv = buf[1:1 + M * D].view(M, D)
    xv.copy_(x)
    assert _ptr(xv) % 16 != 0
    a, b = gdn_ab_projections(xv, wa, wb)
    a_ref, b_ref = gdn_ab_projections(x, wa, wb)
    torch.cuda.synchronize()
    assert torch.equal(a, a_ref) and torch.equal(b, b_ref)


def test_layer_projections_outside_the_kernel_limits_use_library_gemms():
    """Hv above the one-pass kernel's 128 heads (or D not a multiple of 8) goes to F.linear
    in the layer module, bit for bit what the two library GEMMs give."""
    from omegalax_amd.layer import GDNConfig, GDNParams, _projections
    from omegalax_amd.deltanet import ab_proj_supported
    F = torch.nn.functional
    for D, Hv in ((2048, 160), (100, 4)):
        print(f"layer projections fallback D={D} Hv={Hv}", flush=True)
        assert not ab_proj_supported(D, Hv)
        x, wa, wb = inputs(48, D, Hv, D + Hv)
        cfg = GDNConfig(hidden_size=D, num_k_heads=1, head_k_dim=16, num_v_heads=Hv,
                        head_v_dim=16)
        bf = lambda *shape: (0.02 * torch.randn(*shape)).bfloat16().cuda()
        f32 = lambda *shape: torch.zeros(*shape, device="cuda")
        params = GDNParams(in_proj_qkv=bf(cfg.conv_dim, D), in_proj_z=bf(Hv * 16, D),
                           in_proj_b=wb, in_proj_a=wa, conv_w=f32(cfg.conv_dim, 4),
                           dt_bias=f32(Hv), A_log=f32(Hv), norm_w=f32(16),
                           out_proj=bf(D, Hv * 16))
        _, _, a, b = _projections(params, cfg, x)
        torch.cuda.synchronize()
        assert torch.equal(a, F.linear(x, wa)) and torch.equal(b, F.linear(x, wb))
