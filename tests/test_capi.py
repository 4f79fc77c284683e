"""C-ABI tests that need no GPU: the library loads, exports every declared entry
point, and rejects invalid requests on the host before any HIP call."""
import ctypes
import os
import re

import pytest

from omegalax_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "omx_gdn.h")

pytestmark = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH),
                                reason="libomx_gdn.so not built (python -m omegalax_amd.build)")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(omx_gdn_\w+)\s*\(", text)))


def test_header_declares_the_binding_table():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(L, name), name


def test_abi_version():
    assert _lib.lib().omx_gdn_abi_version() == 104


def _decode(**over):
    args = dict(mixed_qkv=1, z=1, a=1, b=1, conv_w=1, A_log=1, dt_bias=1, norm_w=1, eps=1e-6,
                conv_state=1, state=16, out=1, B=2, Hk=2, Hv=4, dk=128, dv=128, K=4, stream=None)
    args.update(over)
    L = _lib.lib()
    rc = L.omx_gdn_decode_step(*args.values())
    return rc, L.omx_gdn_last_error().decode()


@pytest.mark.parametrize("over,code,msg", [
    (dict(Hv=5), _lib.EINVAL, "multiple of key heads"),
    (dict(Hk=0), _lib.EINVAL, "positive"),
    (dict(K=1), _lib.EINVAL, "conv kernel size"),
    (dict(K=9), _lib.EINVAL, "conv kernel size"),
    (dict(B=-1), _lib.EINVAL, "batch"),
    (dict(B=70000), _lib.EINVAL, "batch"),
    (dict(eps=-1.0), _lib.EINVAL, "eps"),
    (dict(dk=96), _lib.EUNSUPPORTED, "not compiled"),
    (dict(Hk=1, Hv=16), _lib.EUNSUPPORTED, "gqa"),
    (dict(state=None), _lib.EINVAL, "NULL"),
    (dict(out=None), _lib.EINVAL, "NULL"),
    (dict(state=8), _lib.EINVAL, "aligned"),
])
def test_decode_rejects_bad_arguments(over, code, msg):
    rc, err = _decode(**over)
    assert rc == code
    assert msg in err


def test_decode_zero_batch_is_a_noop():
    rc, err = _decode(B=0, state=None, out=None)
    assert rc == _lib.OK and err == ""


def test_recurrent_step_rejects_bad_dtype_and_null():
    L = _lib.lib()
    rc = L.omx_gdn_recurrent_step(1, 1, 1, 7, 1, 1, 16, 1, 1, 1, 1, 64, 64, 0.125, None)
    assert rc == _lib.EINVAL and "in_dtype" in L.omx_gdn_last_error().decode()
    rc = L.omx_gdn_recurrent_step(1, 1, None, 0, 1, 1, 16, 1, 1, 1, 1, 64, 64, 0.125, None)
    assert rc == _lib.EINVAL and "NULL" in L.omx_gdn_last_error().decode()


def test_call_raises_gdnerror_with_message():
    with pytest.raises(_lib.GDNError, match="multiple of key heads"):
        _lib.call("omx_gdn_decode_step", 1, 1, 1, 1, 1, 1, 1, 1, 1e-6, 1, 16, 1,
                  1, 3, 4, 128, 128, 4, None)


def test_python_api_rejects_cpu_tensors():
    torch = pytest.importorskip("torch")
    from omegalax_amd import recurrent_gated_delta_rule_step
    q = torch.zeros(1, 1, 16)
    with pytest.raises(ValueError, match="GPU"):
        recurrent_gated_delta_rule_step(q, q, torch.zeros(1, 1, 16), torch.zeros(1, 1),
                                        torch.zeros(1, 1), torch.zeros(1, 1, 16, 16))


def _ws_size(B=2, T=100, Hk=2, Hv=4, dk=128, dv=128, N=2, dt=_lib.BF16):
    return _lib.lib().omx_gdn_chunk_fwd_workspace_size(B, T, Hk, Hv, dk, dv, N, dt)


def test_chunk_workspace_size_covers_records_and_normalised_qk():
    # records: (ceil(B*T/64) + N) slots x Hv x 19 KiB (bf16) or 25 KiB (fp32), plus q/k
    bf, f32 = _ws_size(dt=_lib.BF16), _ws_size(dt=_lib.F32)
    slots = (2 * 100 + 63) // 64 + 2
    assert bf >= slots * 4 * 19456 + 2 * 200 * 2 * 128 * 2
    assert f32 >= slots * 4 * 25600 + 2 * 200 * 2 * 128 * 4
    assert f32 > bf
    assert _ws_size(T=1000) > _ws_size(T=100)
    prefill = _lib.lib().omx_gdn_prefill_workspace_size(2, 100, 2, 4, 128, 128, 2)
    assert prefill > bf  # adds conv(v), bf16 o and the norm's partial sums


def _chunk(ws, ws_bytes, **over):
    a = dict(q=16, k=16, v=16, dt=_lib.BF16, g=16, beta=16, s0=None, cu=None, N=2, o=16, fs=None,
             B=2, T=100, Hk=2, Hv=4, dk=128, dv=128, C=64, scale=0.088, norm=1, ws=ws,
             ws_bytes=ws_bytes, stream=None)
    a.update(over)
    L = _lib.lib()
    rc = L.omx_gdn_chunk_fwd(*a.values())
    return rc, L.omx_gdn_last_error().decode()


@pytest.mark.parametrize("over,msg", [
    (dict(ws_bytes=1024), "workspace"),
    (dict(ws=24), "aligned"),
    (dict(ws=None), "workspace"),
    (dict(C=32), "chunk_size"),
    (dict(dt=5), "in_dtype"),
    (dict(N=3), "N must equal B"),
])
def test_chunk_fwd_rejects_bad_arguments(over, msg):
    args = dict(ws=256, ws_bytes=_ws_size())
    args.update(over)
    rc, err = _chunk(args.pop("ws"), args.pop("ws_bytes"), **args)
    assert rc == _lib.EINVAL
    assert msg in err


def test_prefill_rejects_small_workspace():
    L = _lib.lib()
    need = L.omx_gdn_prefill_workspace_size(2, 100, 2, 4, 128, 128, 2)
    rc = L.omx_gdn_prefill(16, 16, 16, 16, 16, 16, 16, 16, 1e-6, None, 2, None, None, None, None, 16,
                           2, 100, 2, 4, 128, 128, 4, 64, 256, need - 1, None)
    assert rc == _lib.EINVAL and "workspace" in L.omx_gdn_last_error().decode()


def _bwd_ws_size(B=2, T=100, Hk=2, Hv=4, dk=128, dv=128, N=2, dt=_lib.BF16):
    return _lib.lib().omx_gdn_chunk_bwd_workspace_size(B, T, Hk, Hv, dk, dv, N, dt)


def test_bwd_workspace_adds_states_and_chunk_matrices():
    # forward workspace + per (slot, value head): X, Lg, P, G (49,408 B) and two fp32
    # states, plus V_new / dV_new and the per-value-head dq / dk rows
    slots = (2 * 100 + 63) // 64 + 2
    need = (_ws_size() + slots * 4 * 49408 + 2 * slots * 4 * 128 * 128 * 4
            + 2 * 200 * 4 * 128 * 4 + 2 * 200 * 4 * 128 * 4)
    assert _bwd_ws_size() >= need
    assert _bwd_ws_size(T=1000) > _bwd_ws_size(T=100)


def _bwd(ws, ws_bytes, **over):
    a = dict(q=16, k=16, v=16, dt=_lib.BF16, g=16, beta=16, s0=None, cu=None, N=2, do=16, dht=None,
             dq=16, dk=16, dv=16, dg=16, db=16, dh0=None, B=2, T=100, Hk=2, Hv=4, dkd=128, dvd=128,
             C=64, scale=0.088, norm=1, ws=ws, ws_bytes=ws_bytes, stream=None)
    a.update(over)
    L = _lib.lib()
    rc = L.omx_gdn_chunk_bwd(*a.values())
    return rc, L.omx_gdn_last_error().decode()


@pytest.mark.parametrize("over,code,msg", [
    (dict(ws_bytes=1024), _lib.EINVAL, "workspace"),
    (dict(ws=24), _lib.EINVAL, "aligned"),
    (dict(C=32), _lib.EINVAL, "chunk_size"),
    (dict(dt=5), _lib.EINVAL, "in_dtype"),
    (dict(N=3), _lib.EINVAL, "N must equal B"),
    (dict(do=None), _lib.EINVAL, "NULL"),
    (dict(dg=None), _lib.EINVAL, "NULL"),
    (dict(Hv=5), _lib.EINVAL, "multiple of key heads"),
    (dict(dkd=256), _lib.EUNSUPPORTED, "not supported"),
    (dict(dvd=256), _lib.EUNSUPPORTED, "not supported"),
    (dict(dt=_lib.F32), _lib.EUNSUPPORTED, "not supported"),  # fp32 inputs: dk <= 64
    (dict(dkd=96, ws_bytes=_bwd_ws_size()), _lib.EINVAL, "workspace"),  # padded: more workspace
])
def test_chunk_bwd_rejects_bad_arguments(over, code, msg):
    args = dict(ws=256, ws_bytes=_bwd_ws_size())
    args.update(over)
    rc, err = _bwd(args.pop("ws"), args.pop("ws_bytes"), **args)
    assert rc == code
    assert msg in err


def _prefill_bwd(**over):
    L = _lib.lib()
    need = L.omx_gdn_prefill_bwd_workspace_size(2, 100, 2, 4, 128, 128, 2)
    a = dict(x=16, z=16, a=16, b=16, conv_w=16, A_log=16, dt_bias=16, norm_w=16, eps=1e-6, cu=None,
             N=2, s0=None, d_out=16, dht=None, dx=16, dz=16, da=16, db=16, dw=16, dA=16, ddt=16,
             dnw=16, dh0=None, B=2, T=100, Hk=2, Hv=4, dk=128, dv=128, K=4, C=64, ws=256,
             ws_bytes=need, stream=None)
    a.update(over)
    rc = L.omx_gdn_prefill_bwd(*a.values())
    return rc, L.omx_gdn_last_error().decode()


@pytest.mark.parametrize("over,code,msg", [
    (dict(ws_bytes=1024), _lib.EINVAL, "workspace"),
    (dict(K=3), _lib.EINVAL, "conv kernel size must be 4"),
    (dict(z=8), _lib.EINVAL, "16-byte aligned"),
    (dict(d_out=24), _lib.EINVAL, "16-byte aligned"),
    (dict(dz=None), _lib.EINVAL, "NULL"),
    (dict(Hk=1, Hv=257), _lib.EUNSUPPORTED, "Hv <= 256"),
])
def test_prefill_bwd_rejects_bad_arguments(over, code, msg):
    rc, err = _prefill_bwd(**over)
    assert rc == code, err
    assert msg in err


@pytest.mark.parametrize("dk,dv,f32", [(16, 32, False), (96, 80, False), (16, 32, True),
                                       (128, 64, True), (20, 24, True)])
def test_uncompiled_head_dims_run_padded_with_more_workspace(dk, dv, f32):
    """Head dims the kernels are not compiled for run on zero-padded copies: the workspace
    holds the padded buffers on top of the padded call's own workspace."""
    L = _lib.lib()
    dt = _lib.F32 if f32 else _lib.BF16
    dk2 = 32 if (f32 and dk <= 32) else (64 if dk <= 64 else 128)
    dv2 = (dv + 63) // 64 * 64
    direct = L.omx_gdn_chunk_fwd_workspace_size(2, 100, 2, 4, dk2, dv2, 2, dt)
    padded = L.omx_gdn_chunk_fwd_workspace_size(2, 100, 2, 4, dk, dv, 2, dt)
    if (dk2, dv2) == (dk, dv):
        assert padded == direct
    else:
        esz = 4 if f32 else 2
        extra = 200 * (2 * 2 * dk2 + 4 * dv2) * esz + 200 * 4 * dv2 * 4 + 2 * 2 * 4 * dk2 * dv2 * 4
        assert padded >= direct + extra
    if not f32:
        assert (L.omx_gdn_prefill_workspace_size(2, 100, 2, 4, dk, dv, 2)
                > L.omx_gdn_prefill_workspace_size(2, 100, 2, 4, dk2, dv2, 2))


def test_head_dims_beyond_every_compiled_size_are_unsupported():
    L = _lib.lib()
    ws = L.omx_gdn_chunk_fwd_workspace_size(1, 64, 1, 1, 256, 64, 1, _lib.BF16)
    rc, err = _chunk(256, ws, B=1, T=64, N=1, Hk=1, Hv=1, dk=256, dv=64)
    assert rc == _lib.EUNSUPPORTED and "not supported" in err
    ws = L.omx_gdn_chunk_fwd_workspace_size(1, 64, 1, 1, 64, 320, 1, _lib.BF16)
    rc, err = _chunk(256, ws, B=1, T=64, N=1, Hk=1, Hv=1, dk=64, dv=320)
    assert rc == _lib.EUNSUPPORTED and "not supported" in err


def test_prefill_noalloc_rejects_shapes_beyond_its_fixed_scratch():
    """The check runs on the host before any HIP call."""
    L = _lib.lib()
    cap = L.omx_gdn_prefill_noalloc_max_scratch()
    assert cap == 64 << 20
    assert L.omx_gdn_prefill_workspace_size(1, 2429, 16, 32, 128, 128, 1) <= cap
    assert L.omx_gdn_prefill_workspace_size(1, 2430, 16, 32, 128, 128, 1) > cap
    rc = L.omx_gdn_prefill_noalloc(16, 16, 16, 16, 16, 16, 16, 16, 1e-6, None, 1, None, None,
                                   None, None, 16, 1, 4096, 16, 32, 128, 128, 4, 64, None)
    assert rc == _lib.EINVAL
    assert "scratch" in L.omx_gdn_last_error().decode()


@pytest.mark.parametrize("dk,dv", [(128, 128), (16, 32)])  # compiled dims, padded copies
@pytest.mark.parametrize("over,msg", [
    (dict(chunk_size=32), "chunk_size must be 64"),
    (dict(out=None), "NULL"),
    (dict(conv_w=None), "NULL"),
    (dict(K=5), "conv kernel size"),
    (dict(eps=2.0), "eps"),
    (dict(N=2), "N must equal B"),
])
def test_prefill_noalloc_checks_arguments_before_any_hip_call(dk, dv, over, msg):
    """Bad arguments give EINVAL from the host checks alone: on this GPU-less host any HIP
    call (the device query that finds the scratch array included) would fail with
    ELAUNCH instead, so the code proves that nothing ran before the checks."""
    L = _lib.lib()
    args = dict(mixed_qkv=16, z=16, a=16, b=16, conv_w=16, A_log=16, dt_bias=16, norm_w=16,
                eps=1e-6, cu_seqlens=None, N=1, initial_state=None, final_state=None,
                conv_state_in=None, conv_state_out=None, out=16, B=1, T=64, Hk=2, Hv=4, dk=dk,
                dv=dv, K=4, chunk_size=64, stream=None)
    args.update(over)
    rc = L.omx_gdn_prefill_noalloc(*args.values())
    err = L.omx_gdn_last_error().decode()
    assert rc == _lib.EINVAL, (rc, err)
    assert msg in err, err


def test_xla_ffi_handlers_build_only_with_jax():
    """The XLA FFI handler source is built only where jaxlib's FFI headers exist; here (no
    JAX) the build skips it cleanly and the torch path does not need it."""
    from omegalax_amd import build as B
    assert os.path.exists(B.XLA_SRC)
    src = open(B.XLA_SRC).read()
    for name in ("OmxGdnChunkFwd", "OmxGdnChunkBwd", "OmxGdnPrefill", "OmxGdnPrefillBwd",
                 "OmxGdnDecodeStep"):
        assert f"XLA_FFI_DEFINE_HANDLER_SYMBOL({name}," in src
    try:
        import jax  # noqa: F401
    except ImportError:
        assert B.xla_include_dir() is None
        assert B.build_xla_ffi(verbose=False) is None


def test_ab_proj_rejects_bad_shapes_on_the_host():
    L = _lib.lib()
    # D must be a positive multiple of 8; 1 <= Hv <= 128; M = 0 is an empty call
    assert L.omx_gdn_ab_proj(16, 16, 16, 16, 16, 4, 20, 4, None) == _lib.EINVAL
    assert "multiple of 8" in L.omx_gdn_last_error().decode()
    assert L.omx_gdn_ab_proj(16, 16, 16, 16, 16, 4, 64, 0, None) == _lib.EINVAL
    assert L.omx_gdn_ab_proj(16, 16, 16, 16, 16, 4, 64, 129, None) == _lib.EINVAL
    assert L.omx_gdn_ab_proj(None, None, None, None, None, 0, 64, 32, None) == _lib.OK
    assert L.omx_gdn_ab_proj(None, 16, 16, 16, 16, 4, 64, 32, None) == _lib.EINVAL
    assert "NULL" in L.omx_gdn_last_error().decode()
    assert L.omx_gdn_ab_proj(24, 16, 16, 16, 16, 4, 64, 32, None) == _lib.EINVAL
    assert "aligned" in L.omx_gdn_last_error().decode()


def test_qkv_conv_proj_rejects_bad_shapes_on_the_host():
    L = _lib.lib()
    f = L.omx_gdn_qkv_conv_proj
    # (x, w, conv_w, out, M, D, N, T, K, conv, stream)
    assert f(16, 16, 16, 16, 8, 100, 256, 8, 4, 0, None) == _lib.EINVAL  # D not a multiple of 128
    assert "multiple of 128" in L.omx_gdn_last_error().decode()
    assert f(16, 16, 16, 16, 8, 128, 300, 8, 4, 0, None) == _lib.EINVAL  # N not a multiple of 256
    assert "multiple of 256" in L.omx_gdn_last_error().decode()
    assert f(16, 16, 16, 16, 10, 128, 256, 4, 4, 1, None) == _lib.EINVAL  # M not whole sequences
    assert "sequences" in L.omx_gdn_last_error().decode()
    assert f(16, 16, 16, 16, 8, 128, 256, 8, 3, 1, None) == _lib.EINVAL  # K != 4
    assert f(16, 16, 16, 16, 8, 128, 256, 8, 4, 2, None) == _lib.EINVAL
    assert f(16, 16, 16, 16, 1 << 20, 2048, 256, 1, 4, 0, None) == _lib.EINVAL  # x over 2 GiB
    assert f(None, None, None, None, 0, 128, 256, 1, 4, 1, None) == _lib.OK  # empty call
    assert f(16, None, 16, 16, 8, 128, 256, 8, 4, 1, None) == _lib.EINVAL
    assert "NULL" in L.omx_gdn_last_error().decode()
    assert f(16, 16, None, 16, 8, 128, 256, 8, 4, 1, None) == _lib.EINVAL  # conv needs conv_w
    assert f(24, 16, 16, 16, 8, 128, 256, 8, 4, 1, None) == _lib.EINVAL
    assert "aligned" in L.omx_gdn_last_error().decode()
