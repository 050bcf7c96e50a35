"""Paged decode attention (reference ``kitty/kernels/attention.py``).

``paged_attention`` keeps the reference signature (one sequence, page list,
pools, FP16 sinks and Q-buffer tail) and runs the fused split-K HIP kernel on
device tensors, the torch code of ``kernels.cpu`` on CPU tensors (the
reference's dispatch by device, ``kernels/attention.py:320-341``);
``paged_attention_batched`` is the batched entry point (B sequences, int32
page table) that the drop-in module and the benchmark use.
"""
from __future__ import annotations

from typing import List

import torch

from .. import _hip
from . import cpu
from .ops import _need, paged_decode, stage_i32


def paged_attention(q: torch.Tensor, page_list: List[int], key_baseline: torch.Tensor, key_boost: torch.Tensor,
                    key_meta: torch.Tensor, value_pool: torch.Tensor, value_meta: torch.Tensor,
                    boost_idx: torch.Tensor, D_boost: int, sink_k: torch.Tensor, sink_v: torch.Tensor,
                    qbuf_k: torch.Tensor, qbuf_v: torch.Tensor, num_q_heads: int, num_kv_heads: int,
                    head_dim: int) -> torch.Tensor:
    """(num_q_heads, head_dim) fp16 attention output for one decode step.

    Tokens: sinks ‖ dequantised pages ‖ (qbuf_k, qbuf_v) — the tail is
    attended only when qbuf_k is non-empty, and then K and V tails must have
    the same length (attention.py:163-165; the reference fails in its
    broadcast otherwise, which is raised here as RuntimeError)."""
    _need(q.shape == (num_q_heads, head_dim), "q must be (num_q_heads, head_dim)")
    _need(key_boost.shape[2] == D_boost, "D_boost does not match key_boost")
    n_tail = qbuf_k.shape[1]
    if n_tail > 0 and qbuf_v.shape[1] != n_tail:
        raise RuntimeError(f"key tail has {n_tail} tokens but value tail has {qbuf_v.shape[1]}; "
                           "the reference requires equal lengths (attention.py:163-165,186)")
    if q.device.type == "cpu":
        return cpu.paged_attention(q, page_list, key_baseline, key_boost, key_meta, value_pool, value_meta,
                                   boost_idx, D_boost, sink_k, sink_v, qbuf_k, qbuf_v, num_q_heads, num_kv_heads,
                                   head_dim)
    dev = _hip.require_device(q, key_baseline, sink_k, qbuf_k)
    n_sink = sink_k.shape[1]
    # lengths and the page list in one non-blocking copy from pinned staging
    staged = stage_i32([len(page_list), n_sink, n_tail] + (list(page_list) or [0]), dev)
    lens, pages = staged[:3], staged[3:].view(1, -1)
    tail_v = qbuf_v if n_tail > 0 else qbuf_k
    out = paged_decode(q.view(1, num_q_heads, head_dim), pages, lens[0:1], key_baseline, key_boost, key_meta,
                       value_pool, value_meta, boost_idx.contiguous(),
                       sink_k.unsqueeze(0), sink_v.unsqueeze(0), lens[1:2],
                       qbuf_k.unsqueeze(0), tail_v.unsqueeze(0), lens[2:3],
                       max_pages=len(page_list))
    return out.view(num_q_heads, head_dim)


# The reference's name for its CPU path (kernels/attention.py:46-189): the same
# dispatch, so CPU tensors run the torch code and device tensors the kernel.
paged_attention_reference = paged_attention

paged_attention_batched = paged_decode
