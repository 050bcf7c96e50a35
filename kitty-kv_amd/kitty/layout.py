"""Page pool, free list and page table of the Kitty KV cache (HBM-resident).

Drop-in for ``PageCentricKVLayoutManager`` (reference ``kitty/layout.py:75-316``):
the same five pools with the same shapes and the same public methods.

Pools (one physical page = all KV heads of one (sequence, layer, page#)):

    key_baseline   (P, H, D, G/4)   uint8    low 2 bits of every channel
    key_boost      (P, H, Dk, G/4)  uint8    high 2 bits of boosted channels
    key_metadata   (P, H, 2, D)     dtype    row 0 scale, row 1 zero point
    value_pool     (P, H, G, D/4)   uint8    4 channels per byte
    value_metadata (P, H, G, 2)     dtype    per-token (scale, zero point)

At D = G = 128 a (page, head) record is 9,728 B (12.5% boost) or 10,240 B
(25%); the pools are addressed with int32 page ids and 64-bit byte offsets
in the kernels, so P may grow to the ~3.7 M pages that fill the 288 GB of an
MI355X.  dtype is the config's (float16 or bfloat16, layout.py:123-137); a
bfloat16 pool holds the fp16 scale converted to bfloat16, as the reference
copies it.

Allocation is first-fit on the lowest free index, as the reference's
``free_mask.nonzero()[0]`` (layout.py:186-188), but O(log n) without a device
sync: indices at or above a high-water mark are free, and freed indices below
it sit in a min-heap.
"""
from __future__ import annotations

import heapq
from dataclasses import dataclass
from itertools import repeat
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import torch

from .config import KittyConfig


@dataclass
class Page:
    """A quantised page of G tokens (reference layout.py:44-68)."""

    physical_idx: int
    layer_id: int
    head_id: int
    seq_id: int
    start_token: int
    num_tokens: int = 0

    def __repr__(self) -> str:
        return (f"Page(phys={self.physical_idx}, layer={self.layer_id}, head={self.head_id}, "
                f"seq={self.seq_id}, tokens=[{self.start_token}..{self.start_token + self.num_tokens}))")


class PageCentricKVLayoutManager:
    """Pre-allocated HBM pools + free list + page table."""

    def __init__(self, config: KittyConfig, boost_idx_uint8: torch.Tensor) -> None:
        self.config = config
        self.boost_idx_uint8 = boost_idx_uint8.to(config.device)
        G, D, K, H = config.q_buffer_size, config.head_dim, config.d_boost, config.num_kv_heads
        P = config.pool_pages
        dev = torch.device(config.device)
        self._torch_dtype = torch.float16 if config.dtype == "float16" else torch.bfloat16

        self.key_baseline = torch.zeros(P, H, D, G // 4, dtype=torch.uint8, device=dev)
        self.key_boost = torch.zeros(P, H, K, G // 4, dtype=torch.uint8, device=dev)
        self.key_metadata = torch.zeros(P, H, 2, D, dtype=self._torch_dtype, device=dev)
        self.value_pool = torch.zeros(P, H, G, D // 4, dtype=torch.uint8, device=dev)
        self.value_metadata = torch.zeros(P, H, G, 2, dtype=self._torch_dtype, device=dev)

        self._num_pages_total = P
        self._high_water = 0
        self._freed: List[int] = []
        self._num_free = P
        self._page_table: Dict[Tuple[int, int, int], int] = {}
        self._seq_keys: Dict[int, set] = {}  # seq_id -> its (layer, page number) entries of the page table

    # ------------------------------------------------------------ allocation
    def _pop_lowest_free(self) -> int:
        if self._freed:
            return heapq.heappop(self._freed)
        idx = self._high_water
        self._high_water += 1
        return idx

    def allocate_page(self, seq_id: int, layer_id: int, page_number: int) -> Page:
        """Allocate the lowest free physical page; RuntimeError when exhausted
        (reference layout.py:161-203)."""
        if self._num_free == 0:
            raise RuntimeError(
                "KV Cache page pool exhausted! "
                f"All {self._num_pages_total} pages are in use. "
                "Increase config.max_pages or reduce max_seq_len/max_batch_size.")
        phys = self._pop_lowest_free()
        self._num_free -= 1
        self._page_table[(seq_id, layer_id, page_number)] = phys
        self._seq_keys.setdefault(seq_id, set()).add((layer_id, page_number))
        return Page(physical_idx=phys, layer_id=layer_id, head_id=-1, seq_id=seq_id,
                    start_token=page_number * self.config.q_buffer_size)

    def allocate_run(self, seq_id: int, layer_id: int, first_page: int, count: int) -> List[int]:
        """Physical pages for page numbers first_page .. first_page + count - 1
        of one (sequence, layer), each the lowest free page as count
        allocate_page calls would give, all or nothing."""
        if count > self._num_free:
            raise RuntimeError(
                "KV Cache page pool exhausted! "
                f"{self._num_free} free pages, {count} needed.")
        freed = self._freed
        if len(freed) <= count:
            # every freed index is below the high-water mark: the lowest
            # `count` free pages are all of them, in order, then a fresh run
            phys = sorted(freed)
            freed.clear()
            hw = self._high_water
            self._high_water = hw + count - len(phys)
            phys.extend(range(hw, self._high_water))
        elif count <= 8:
            phys = [heapq.heappop(freed) for _ in range(count)]
        else:
            freed.sort()            # a sorted list is still a min-heap: take its head
            phys = freed[:count]
            del freed[:count]
        self._num_free -= count
        numbers = range(first_page, first_page + count)
        self._page_table.update(zip(zip(repeat(seq_id), repeat(layer_id), numbers), phys))
        self._seq_keys.setdefault(seq_id, set()).update(zip(repeat(layer_id), numbers))
        return phys

    def allocate_pages(self, seq_id: int, layer_ids: Sequence[int], page_number: int) -> List[int]:
        """Allocate one page per layer for a spill; all-or-nothing."""
        if self._num_free < len(layer_ids):
            raise RuntimeError(
                "KV Cache page pool exhausted! "
                f"{self._num_free} free pages, {len(layer_ids)} needed.")
        return [self.allocate_page(seq_id, l, page_number).physical_idx for l in layer_ids]

    def free_page(self, seq_id: int, layer_id: int, page_number: int) -> None:
        phys = self._page_table.pop((seq_id, layer_id, page_number), None)
        if phys is None:
            return
        keys = self._seq_keys.get(seq_id)
        if keys is not None:
            keys.discard((layer_id, page_number))
        heapq.heappush(self._freed, phys)
        self._num_free += 1

    def free_sequence(self, seq_id: int) -> None:
        for layer_id, page_number in sorted(self._seq_keys.pop(seq_id, ())):
            phys = self._page_table.pop((seq_id, layer_id, page_number))
            heapq.heappush(self._freed, phys)
            self._num_free += 1

    def get_physical_idx(self, seq_id: int, layer_id: int, page_number: int) -> int:
        key = (seq_id, layer_id, page_number)
        if key not in self._page_table:
            raise KeyError(f"Page {key} not found in page table.")
        return self._page_table[key]

    # ------------------------------------------------------------- accessors
    def key_baseline_page(self, phys_idx: int) -> torch.Tensor:
        return self.key_baseline[phys_idx]

    def key_boost_page(self, phys_idx: int) -> torch.Tensor:
        return self.key_boost[phys_idx]

    def key_meta_page(self, phys_idx: int) -> torch.Tensor:
        return self.key_metadata[phys_idx]

    def value_page(self, phys_idx: int) -> torch.Tensor:
        return self.value_pool[phys_idx]

    def value_meta_page(self, phys_idx: int) -> torch.Tensor:
        return self.value_metadata[phys_idx]

    # ------------------------------------------------------------ page lists
    def get_page_list(self, seq_id: int, layer_id: int) -> List[int]:
        pages = []
        n = 0
        while (seq_id, layer_id, n) in self._page_table:
            pages.append(self._page_table[(seq_id, layer_id, n)])
            n += 1
        return pages

    def block_table(self, seq_ids: Iterable[int], layer_id: int,
                    device: Optional[torch.device] = None) -> Tuple[torch.Tensor, torch.Tensor, int]:
        """Page-table indirection for a batched decode step: int32 (B, max_pages)
        physical ids, int32 (B,) page counts, and max_pages."""
        lists = [self.get_page_list(s, layer_id) for s in seq_ids]
        width = max([len(l) for l in lists] + [1])
        bt = torch.zeros(len(lists), width, dtype=torch.int32)
        for i, l in enumerate(lists):
            if l:
                bt[i, :len(l)] = torch.tensor(l, dtype=torch.int32)
        n = torch.tensor([len(l) for l in lists], dtype=torch.int32)
        dev = device if device is not None else self.key_baseline.device
        return bt.to(dev), n.to(dev), max([len(l) for l in lists] + [0])

    # ----------------------------------------------------------------- stats
    def memory_stats(self) -> Dict[str, float]:
        def mb(t: torch.Tensor) -> float:
            return t.numel() * t.element_size() / (1024 ** 2)

        pools = [self.key_baseline, self.key_boost, self.key_metadata, self.value_pool, self.value_metadata]
        return {
            "key_baseline_MB": mb(self.key_baseline),
            "key_boost_MB": mb(self.key_boost),
            "key_metadata_MB": mb(self.key_metadata),
            "value_pool_MB": mb(self.value_pool),
            "value_metadata_MB": mb(self.value_metadata),
            "total_MB": sum(mb(t) for t in pools),
            "pages_free": self._num_free,
            "pages_used": self._num_pages_total - self._num_free,
            "pages_total": self._num_pages_total,
        }

    def __repr__(self) -> str:
        s = self.memory_stats()
        return (f"PageCentricKVLayoutManager(\n"
                f"  key_baseline:  {tuple(self.key_baseline.shape)}  uint8\n"
                f"  key_boost:     {tuple(self.key_boost.shape)}  uint8\n"
                f"  key_metadata:  {tuple(self.key_metadata.shape)}  {self.key_metadata.dtype}\n"
                f"  value_pool:    {tuple(self.value_pool.shape)}  uint8\n"
                f"  value_metadata:{tuple(self.value_metadata.shape)}  {self.value_metadata.dtype}\n"
                f"  Pages: {s['pages_used']}/{s['pages_total']} used ({s['total_MB']:.1f} MB total)\n)")
