"""Host-side plumbing around the kernels that needs no GPU: packed-document
metadata (segment ids -> cu_seqlens), right-pad lengths, and the Hugging Face
checkpoint mapping of the GDN parameters (loader.py:173-190, 226-307)."""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from omegalax_amd.segments import lengths_to_cu_seqlens, right_pad_lengths, segment_ids_to_cu_seqlens


def brute_runs(seg):
    """Runs of equal ids along each row, by explicit iteration (the definition)."""
    B, T = seg.shape
    cu = [0]
    for b in range(B):
        for t in range(T):
            if t > 0 and seg[b, t] != seg[b, t - 1]:
                cu.append(b * T + t)
        cu.append((b + 1) * T)
    # row ends coincide with the next row's start: drop duplicates, keep order
    out = []
    for c in cu:
        if not out or out[-1] != c:
            out.append(c)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_segment_ids_to_cu_seqlens_matches_runs(seed):
    rng = np.random.default_rng(seed)
    B, T = int(rng.integers(1, 4)), int(rng.integers(1, 40))
    # packed documents: increasing ids with right padding (id 0), as SFT packing makes them
    seg = np.zeros((B, T), np.int64)
    for b in range(B):
        t, doc = 0, 1
        stop = int(rng.integers(0, T + 1))
        while t < stop:
            n = int(rng.integers(1, 8))
            seg[b, t:min(stop, t + n)] = doc
            t += n
            doc += 1
    cu = segment_ids_to_cu_seqlens(torch.from_numpy(seg))
    assert cu.dtype == torch.int32
    assert cu.tolist() == brute_runs(seg)


def test_segment_ids_row_boundaries_split_equal_ids():
    seg = torch.tensor([[1, 1, 1], [1, 1, 0]])
    assert segment_ids_to_cu_seqlens(seg).tolist() == [0, 3, 5, 6]


def test_right_pad_lengths():
    pad = 7
    ids = torch.tensor([[1, 2, 3, 7, 7], [7, 7, 7, 7, 7], [4, 7, 5, 6, 9], [7, 1, 7, 7, 7]])
    assert right_pad_lengths(ids, pad).tolist() == [3, 0, 5, 2]


def test_lengths_to_cu_seqlens():
    assert lengths_to_cu_seqlens(torch.tensor([3, 0, 5])).tolist() == [0, 3, 3, 8]


def _random_params(rng, D=32, Hk=2, dk=16, Hv=4, dv=16, K=4):
    from omegalax_amd.layer import GDNParams
    C = 2 * Hk * dk + Hv * dv
    t = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32))
    return GDNParams(in_proj_qkv=t(C, D).bfloat16(), in_proj_z=t(Hv * dv, D).bfloat16(),
                     in_proj_b=t(Hv, D).bfloat16(), in_proj_a=t(Hv, D).bfloat16(),
                     conv_w=t(C, K), dt_bias=t(Hv), A_log=t(Hv), norm_w=t(dv),
                     out_proj=t(D, Hv * dv).bfloat16())


def test_hf_mapping_round_trip_through_safetensors(tmp_path):
    pytest.importorskip("safetensors")
    from safetensors.torch import save_file
    from omegalax_amd.layer import gdn_params_to_hf, load_gdn_layers
    rng = np.random.default_rng(0)
    p3, p7 = _random_params(rng), _random_params(rng)
    tensors = {**gdn_params_to_hf(p3, 3), **gdn_params_to_hf(p7, 7)}
    # the checkpoint stores conv1d.weight as [C, 1, K] (loader.py:289 squeezes it)
    assert tensors["model.language_model.layers.3.linear_attn.conv1d.weight"].shape == (p3.conv_w.shape[0], 1, 4)
    path = os.path.join(tmp_path, "gdn.safetensors")
    save_file({k: v.contiguous() for k, v in tensors.items()}, path)
    loaded = load_gdn_layers(path, [3, 7], device="cpu")
    for want, got in ((p3, loaded[3]), (p7, loaded[7])):
        for name in want.__dataclass_fields__:
            assert torch.equal(getattr(want, name), getattr(got, name)), name


def test_hf_mapping_reports_missing_keys():
    from omegalax_amd.layer import gdn_params_from_hf
    with pytest.raises(KeyError, match="conv1d"):
        gdn_params_from_hf({}, 0)


def test_ab_projection_limits_are_checked_up_front():
    """The one-pass gate projection kernel takes D a multiple of 8 and 1 <= Hv <= 128; the
    Python wrapper names the limit before any device work (CPU tensors suffice here)."""
    import torch
    from omegalax_amd.deltanet import _ab_proj_fwd, ab_proj_supported
    assert ab_proj_supported(2048, 32) and ab_proj_supported(8, 128)
    assert not ab_proj_supported(2044, 32) and not ab_proj_supported(2048, 129)
    x = torch.zeros(4, 20, dtype=torch.bfloat16)
    w = torch.zeros(4, 20, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiple of 8"):
        _ab_proj_fwd(x, w, w)
