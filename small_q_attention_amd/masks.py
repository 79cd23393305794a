"""Packed speculative-decoding (draft) masks.

Format of the reference's FlashInfer comparisons
(``/root/reference/scripts/run_flashinfer_baseline.py:56-85``,
``scripts/compare_flashinfer_paths.py:33-46``): for each sequence ``b`` and draft
row ``qi``, ``ceil(Q / 32)`` little-endian 32-bit words whose bit ``j % 32`` of word
``j // 32`` says that row ``qi`` sees draft token ``j`` (the token at position
``seq_len - Q + j``); stored as a ``[B, Q, 2 * ceil(Q / 32)]`` uint16 tensor. Tokens
before the draft block are always visible. The kernels read the same bytes as
``[B, Q, ceil(Q / 32)]`` 32-bit words (:func:`as_words`).
"""

from __future__ import annotations


def _words(q_len: int) -> int:
    return (q_len + 31) // 32


def pack_draft_mask(visible):
    """bool ``[B, Q, Q]`` (row qi sees draft token j) -> packed uint16 ``[B, Q, 2W]``."""
    import torch

    if visible.dim() != 3 or visible.shape[1] != visible.shape[2]:
        raise ValueError("visible must be [B, Q, Q]")
    b, q_len, _ = visible.shape
    w = _words(q_len)
    pad = w * 32 - q_len
    v = visible.to(torch.bool)
    if pad:
        v = torch.cat([v, torch.zeros(b, q_len, pad, dtype=torch.bool, device=v.device)], dim=2)
    v = v.view(b, q_len, w, 32).to(torch.int64)
    weights = torch.tensor([1 << i for i in range(32)], dtype=torch.int64, device=v.device)
    words = (v * weights).sum(-1)  # [B, Q, W], 0 <= x < 2^32
    lo = (words & 0xFFFF).to(torch.int32)
    hi = (words >> 16).to(torch.int32)
    halves = torch.stack([lo, hi], dim=-1).view(b, q_len, 2 * w)
    return halves.to(torch.int32).to(torch.uint16) if hasattr(torch, "uint16") else halves


def spec_dec_mask(batch: int, q_len: int, mode: str = "causal", device=None):
    """The reference's mask builder: ``"causal"`` (row qi sees draft tokens j <= qi) or
    ``"full"`` (every draft token), the same for every sequence."""
    import torch

    qi = torch.arange(q_len, device=device).unsqueeze(1)
    j = torch.arange(q_len, device=device).unsqueeze(0)
    if mode == "causal":
        visible = j <= qi
    elif mode == "full":
        visible = torch.ones(q_len, q_len, dtype=torch.bool, device=device)
    else:
        raise ValueError(f"unsupported spec-dec mask mode: {mode}")
    return pack_draft_mask(visible.unsqueeze(0).expand(batch, q_len, q_len))


def as_words(mask, batch: int, q_len: int):
    """Packed mask (uint16 ``[B, Q, 2W]`` or 32-bit ``[B, Q, W]``) -> contiguous int32
    ``[B, Q, W]`` holding the same bits, on the mask's device."""
    import torch

    w = _words(q_len)
    m = mask.contiguous()
    if m.element_size() == 2:
        if m.shape[-1] % 2:
            raise ValueError("a uint16 draft mask needs an even last dimension")
        m = m.view(torch.int16).view(torch.int32)
    elif m.element_size() == 4:
        m = m.view(torch.int32)
    else:
        raise ValueError("draft mask must hold 16- or 32-bit elements")
    if tuple(m.shape[:2]) != (batch, q_len) or m.shape[2] < w:
        raise ValueError(f"draft mask must be [{batch}, {q_len}, {2 * w}] uint16 "
                         f"(or [{batch}, {q_len}, {w}] 32-bit words)")
    return m[..., :w].contiguous()
