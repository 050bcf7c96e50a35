"""KittyConfig — hyper-parameters and derived constants of the Kitty KV cache.

Same fields, defaults, derived properties, JSON format and validation as the
reference's ``kitty/config.py:18-152`` so that configs saved by either
implementation load in the other.  Derived constants (``config.py:86-110``):

* ``d_boost = round(boost_rate * head_dim)`` (Python's round-half-to-even),
* ``sentinel = min(d_boost + 1, 255)``,
* ``max_pages = ((max_seq_len - sink_size) // q_buffer_size + 2) * max_batch_size``.

The layout manager allocates ``pool_pages`` physical pages, which is
``max_pages`` unless ``pool_pages_override`` is set.  ``max_pages`` ignores
``num_layers`` exactly as the reference does, although every spill takes one
page per layer (``pipeline.py:202-206``); set ``pool_pages_override`` (for
example to ``max_pages * num_layers``) to size a multi-layer pool.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Literal, Optional


@dataclass
class KittyConfig:
    num_layers: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128

    sink_size: int = 32            # S  — FP16 attention sinks
    q_buffer_size: int = 128       # G  — tokens per quantised page / key Q-buffer
    local_value_window: int = 128  # R  — FP16 value window

    boost_rate: float = 0.125      # 0.125 Kitty, 0.25 Kitty-Pro

    max_seq_len: int = 32768
    max_batch_size: int = 1
    dtype: Literal["float16", "bfloat16"] = "float16"
    device: str = "cuda:0"

    profile_save_dir: str = "kitty_profiles"
    variant: Literal["kitty", "kitty-pro"] = "kitty"

    # Physical pool size in pages; None means max_pages, as in the reference.
    pool_pages_override: Optional[int] = None

    @property
    def d_boost(self) -> int:
        return round(self.boost_rate * self.head_dim)

    @property
    def max_pages(self) -> int:
        per_seq = (self.max_seq_len - self.sink_size) // self.q_buffer_size + 2
        return per_seq * self.max_batch_size

    @property
    def sentinel(self) -> int:
        return min(self.d_boost + 1, 255)

    @property
    def pool_pages(self) -> int:
        """Physical pages allocated by the layout manager."""
        if self.pool_pages_override is not None:
            return int(self.pool_pages_override)
        return self.max_pages

    def save(self, path: str | Path) -> None:
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        data = asdict(self)
        if data.get("pool_pages_override") is None:
            data.pop("pool_pages_override")  # keep the reference's JSON schema
        with open(path, "w") as f:
            json.dump(data, f, indent=2)

    @classmethod
    def load(cls, path: str | Path) -> "KittyConfig":
        with open(path) as f:
            return cls(**json.load(f))

    @classmethod
    def kitty_pro(cls, **kwargs) -> "KittyConfig":
        return cls(boost_rate=0.25, variant="kitty-pro", **kwargs)

    def __post_init__(self) -> None:
        assert 0 < self.boost_rate < 1, "boost_rate must be in (0, 1)"
        assert self.head_dim % 4 == 0, "head_dim must be divisible by 4 (packing)"
        assert self.q_buffer_size % 4 == 0, "q_buffer_size (G) must be divisible by 4 (uint8 packing)"
        assert self.sink_size >= 0
        assert self.local_value_window >= 0
        assert self.dtype in ("float16", "bfloat16")

    def __repr__(self) -> str:
        return (f"KittyConfig(variant={self.variant!r}, num_layers={self.num_layers}, "
                f"num_kv_heads={self.num_kv_heads}, head_dim={self.head_dim}, "
                f"boost_rate={self.boost_rate} -> d_boost={self.d_boost}, "
                f"G={self.q_buffer_size}, S={self.sink_size}, R={self.local_value_window})")
