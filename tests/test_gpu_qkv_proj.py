"""GPU parity of the prototype in_proj_qkv GEMM with the causal conv + SiLU in its
epilogue (omx_gdn_qkv_conv_proj; reference deltanet.py:234-243).

- The plain GEMM (conv = 0) against the fp32 product of the same bf16 inputs, rounded
  to bf16: 1e-2 of the output's scale, about two bf16 ulps (two fp32 accumulation
  orders may round a value to neighbouring bf16 numbers).
- The conv epilogue (conv = 1) against the oracle's conv + SiLU with the reference's
  bf16 rounding points (oracle.gdn_oracle._conv_silu) applied to the kernel's own plain
  output, so the epilogue alone is under test: 1e-2.  Each sequence of T rows starts
  from zeros (deltanet.py:46), which the tests cross at tile and sequence boundaries.
"""
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-2


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def inputs(M, D, N, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(M, D, generator=g, device="cuda").bfloat16()
    w = (torch.randn(N, D, generator=g, device="cuda") / D ** 0.5).bfloat16()
    cw = (0.5 * torch.randn(N, 4, generator=g, device="cuda")).float()
    return x, w, cw


def conv_ref(raw, cw, T, rows):
    """The oracle's conv + SiLU of the bf16 rows `raw` [M, N] (sequences of T rows) at the
    output rows `rows` (a sorted array), each from its own sequence's earlier rows."""
    raw = np.asarray(raw, np.float32)
    out = np.empty((len(rows), raw.shape[1]))
    for i, t in enumerate(rows):
        s = (t // T) * T
        lo = max(s, t - 3)
        hist = None
        if t - 3 < s:  # rows before the sequence start are zeros
            hist = np.zeros((1, raw.shape[1], 3), np.float32)
            k = t - lo  # rows of the window inside the sequence, before t
            if k:
                hist[0, :, 3 - k:] = raw[lo:t].T
            seg = raw[t:t + 1][None]
        else:
            hist = raw[t - 3:t].T[None]
            seg = raw[t:t + 1][None]
        out[i] = O._conv_silu(seg, cw, hist, O.round_bf16)[0, 0]
    return out


def proj(x, w, cw=None, T=None):
    from omegalax_amd import qkv_conv_projection
    y = qkv_conv_projection(x, w, cw, seq_len=T)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("M,D,N", [(300, 256, 512), (1, 128, 256), (513, 384, 768)])
def test_qkv_proj_plain_matches_fp32_product(M, D, N):
    say(f"qkv proj plain M={M} D={D} N={N}")
    x, w, _ = inputs(M, D, N, seed=M + D)
    y = proj(x, w)
    ref = (x.float() @ w.float().T).bfloat16().float()
    assert rel(y.float().cpu().numpy(), ref.cpu().numpy()) < TOL


@pytest.mark.parametrize("B,T,D,N", [(3, 100, 256, 512), (2, 300, 128, 256), (1, 5, 256, 256)])
def test_qkv_conv_epilogue_matches_oracle(B, T, D, N):
    """Sequences shorter than a tile, crossing tiles (T=300 over 256-row tiles) and
    shorter than the conv window's history at the start."""
    say(f"qkv conv B={B} T={T} D={D} N={N}")
    x, w, cw = inputs(B * T, D, N, seed=7 * T + N)
    raw = proj(x, w)
    y = proj(x, w, cw, T)
    rows = np.arange(B * T)
    ref = conv_ref(raw.float().cpu().numpy(), cw.cpu().numpy(), T, rows)
    assert rel(y.float().cpu().numpy(), ref) < TOL


def test_qkv_conv_c1_full_size():
    """C1's in_proj_qkv: 4 sequences of 4096 tokens, D=2048, N=8192.  The plain GEMM
    against the library's (F.linear) on every row; the conv epilogue against the
    oracle on rows at the start, the tile and sequence boundaries and the end."""
    B, T, D, N = 4, 4096, 2048, 8192
    say("qkv conv C1 full size")
    x, w, cw = inputs(B * T, D, N, seed=2048)
    raw = proj(x, w)
    lib = torch.nn.functional.linear(x, w)
    torch.cuda.synchronize()
    err = ((raw.float() - lib.float()).abs().max() / lib.float().abs().max()).item()
    assert err < TOL
    y = proj(x.reshape(B, T, D), w, cw).reshape(B * T, N)
    rows = np.array(sorted({0, 1, 2, 3, 255, 256, 257, 4093, 4094, 4095, 4096, 4097, 4098, 4099,
                            8191, 8192, 12287, 12288, 12290, 16381, 16383}))
    raw_np = raw.float().cpu().numpy()
    ref = conv_ref(raw_np, cw.cpu().numpy(), T, rows)
    assert rel(y.float().cpu().numpy()[rows], ref) < TOL
