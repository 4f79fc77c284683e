"""Packed-document metadata for the varlen prefill.

The reference feeds a packed SFT row through the layer as one sequence, so the
recurrent state and the conv window run on from one document into the next
(omegalax/models/qwen3_5/deltanet.py:227-228 only zeroes padding; model.py:294
passes the segment ids to attention alone).  Here every maximal run of one
segment id within a row becomes its own sequence of the varlen prefill, so both
reset at each document boundary.  Padding (segment id 0, as text/api.py:120 makes
it) forms runs of its own, whose outputs the caller ignores.
"""
from __future__ import annotations

import torch


def segment_ids_to_cu_seqlens(segment_ids_BT: torch.Tensor) -> torch.Tensor:
    """[B, T] segment ids -> int32 cu_seqlens over the flattened B*T tokens.

    A sequence starts at every row start and wherever the id changes along a row;
    the runs tile [0, B*T) in order.  The result lives on the ids' device.
    """
    if segment_ids_BT.dim() != 2:
        raise ValueError("segment_ids must be [B, T]")
    B, T = segment_ids_BT.shape
    dev = segment_ids_BT.device
    if B * T == 0:
        return torch.zeros(1, dtype=torch.int32, device=dev)
    s = segment_ids_BT.to(torch.int64)
    start = torch.ones((B, T), dtype=torch.bool, device=dev)
    start[:, 1:] = s[:, 1:] != s[:, :-1]
    pos = torch.nonzero(start.reshape(-1), as_tuple=False).flatten()
    end = torch.tensor([B * T], dtype=pos.dtype, device=dev)
    return torch.cat([pos, end]).to(torch.int32)


def right_pad_lengths(token_ids_BT: torch.Tensor, pad_id: int) -> torch.Tensor:
    """Valid length of each right-padded row: T minus its trailing pad tokens
    (per row; text/api.py:137 and qwen3/utils.py:10-16 take the batch maximum)."""
    B, T = token_ids_BT.shape
    is_pad = token_ids_BT == pad_id
    # trailing pads = index of the first non-pad from the right
    flipped = torch.flip(~is_pad, dims=[1]).to(torch.int32)
    any_tok = flipped.any(dim=1)
    trailing = torch.where(any_tok, torch.argmax(flipped, dim=1), torch.full_like(any_tok, T, dtype=torch.int64))
    return (T - trailing).to(torch.int32)


def lengths_to_cu_seqlens(lengths: torch.Tensor) -> torch.Tensor:
    """Per-sequence lengths -> int32 cu_seqlens [N+1]."""
    cu = torch.zeros(lengths.numel() + 1, dtype=torch.int64, device=lengths.device)
    cu[1:] = torch.cumsum(lengths.to(torch.int64), dim=0)
    return cu.to(torch.int32)
