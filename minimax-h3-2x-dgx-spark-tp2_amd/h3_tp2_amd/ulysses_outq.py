"""The out projection's per-token FP8 quant read straight from the Ulysses receive buffer, on MI355X.

Mirrors the compute of the reference's h3_tp2/ulysses_outq.py -- ``quant_rows`` (:109-124), ``quant_reference_eager``
(:127-135, the arithmetic) and ``quant_from_recv`` (:138-143): the reverse all-to-all's receive buffer [P, M, hl, d]
holds row m of source p at recv[p, m]; the out projection's input row m is [recv[0, m], ..., recv[P-1, m]], and the
quant reads those P segments in place (``h3fp8_quant_segments``) instead of unpacking them first.  With P = 1 it is
kernel 1.  The deferred-placeholder machinery that routes the out projection's quant here sits in the multi-GPU
exchange and is not part of this single-GPU build.
"""
from __future__ import annotations

import torch

from . import ops

FP8_MAX = ops.FP8_MAX
MIN_SCALE = ops.MIN_SCALE


def quant_rows(base: torch.Tensor, m: int, p: int, seg: int, stride_p: int, stride_m: int):
    """Per-token FP8 quant of M rows whose row m is the P segments ``base[p*stride_p + m*stride_m : +seg]`` (element
    offsets from ``base``'s data pointer; ``base`` bf16 contiguous): (q [M, P*seg] e4m3fn, scale [M, 1] fp32)."""
    return ops.quant_segments(base, m, p, seg, stride_p, stride_m)


def quant_from_recv(recv: torch.Tensor):
    """recv [P, M, hl, d] contiguous -> the quant of the [M, P*hl*d] tensor the unpack would have produced."""
    return ops.quant_from_recv(recv)
