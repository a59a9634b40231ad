"""Drop-in for the reference's ``src/triton_kernels/ssd_chunked_scan.py`` on
the integer MI355X path (forward only).

``ssd_chunked_scan_forward(u, nums, shifts, chunk_size)`` keeps the
reference's contract (``:382-422``): u and nums are [B, L, D], the shift is
read from ``shifts`` (the reference takes its first element, ``:406-409``),
and the result is ``(h, final_h, decay_to_end)`` with ``final_h`` and
``decay_to_end`` of shape [B, ceil(L / chunk_size), D].  The arithmetic is
the integer recurrence of spec mi-spec-2:

- ``h[t] = sat32(floor(h[t-1] * nums[t] / 2^shift) + u[t])`` on int32 u;
- ``final_h`` is the state at the last step of each chunk;
- ``decay_to_end`` is the chunk's cumulative decay prod(nums / 2^shift),
  float32 as in the reference (``:400``): the kernel's Q30 int32 (the floor
  recurrence applied to 2^30 with zero input, rounded down after every step)
  divided by 2^30.  ``mamba_int.ops.dyadic_chunked_scan`` returns the Q30
  integers themselves.

The reference's float recurrence (``h = decay * h + u``, ``:366``) has no
floor; the integer one is not associative, so chunks only bound the outputs
and the state is carried from chunk to chunk in order, as the reference's
kernel carries ``h_prev`` (``:356-379``).  Everything runs in
``mi_dyadic_chunked_scan`` (libmamba_int.so).
"""
from __future__ import annotations

from typing import Tuple, Union

import torch

from mamba_int import ops


def _shift(shifts: Union[int, torch.Tensor]) -> int:
    if not isinstance(shifts, torch.Tensor):
        return int(shifts)
    if shifts.numel() == 0:
        return 15                                   # the reference's default (:407-409)
    flat = shifts.reshape(-1)
    s = int(flat[0].item())
    if not bool((flat == s).all()):
        # the reference silently uses shifts[0] for every element; a mixed
        # tensor would give results that match neither form
        raise ValueError("ssd_chunked_scan_forward: the integer scan takes one shift for the whole tensor")
    return s


def ssd_chunked_scan_forward(u: torch.Tensor, nums: torch.Tensor, shifts, chunk_size: int = 64
                             ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(h, final_h, decay_to_end) of the chunked integer scan; u int32 [B, L, D],
    nums any integer dtype [B, L, D] (converted to int32 as the reference's
    ``SSDChunkedScanFunction.forward`` does, ``:543-544``)."""
    if u.dtype != torch.int32:
        raise TypeError("the integer chunked scan takes int32 u")
    if nums.is_floating_point():
        raise TypeError("the integer chunked scan takes integer decay numerators")
    h, final_h, dte_q30 = ops.dyadic_chunked_scan(u.contiguous(), nums.to(torch.int32).contiguous(),
                                                  _shift(shifts), int(chunk_size))
    return h, final_h, dte_q30.to(torch.float32) * (1.0 / (1 << 30))


class SSDChunkedScanFunction:
    """``SSDChunkedScanFunction.apply(u, nums, shifts, chunk_size)`` (``:537-560``),
    forward only: returns h."""

    @staticmethod
    def apply(u: torch.Tensor, nums: torch.Tensor, shifts, chunk_size: int = 64) -> torch.Tensor:
        return ssd_chunked_scan_forward(u, nums, shifts, chunk_size)[0]


def ssd_chunked_scan(u: torch.Tensor, nums: torch.Tensor, shifts, chunk_size: int = 64) -> torch.Tensor:
    """``ssd_chunked_scan(u, nums, shifts, chunk_size)`` (``:563-583``): h only."""
    return SSDChunkedScanFunction.apply(u, nums, shifts, chunk_size)
