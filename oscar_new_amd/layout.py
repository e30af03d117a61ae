"""Byte geometry of OSCAR's INT2 slots and BF16 windows inside the native K/V stripes.

Host mirror of ``oscar_ascend/layout.py`` (reference). The device kernels evaluate the same
formulas; nothing here allocates memory.

Per physical page (``Bp`` tokens, ``H`` kv heads, ``D`` = 256):

* K stripe page (``stripe_page_bytes = Bp*H*D*2`` bytes) holds INT2 history slots:
  slot ``s`` of head ``h`` starts at ``(s // Bp) * stripe + ((s % Bp) * H + h) * 160``;
  bytes [0,64) K codes, [64,66) K scale (fp16 LE), [66,68) K zero, [68,132) V codes,
  [132,134) V scale, [134,136) V zero, [136,160) untouched padding.
* V stripe page of a request's FIRST physical page holds the BF16 window: sink tokens
  ``t < S`` at index ``t``, later tokens at ring index ``S + t % C``; each index stores K
  then V, ``H*D`` bf16 each.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from .config import OscarConfig


@dataclass(frozen=True)
class CacheLayout:
    """Reference: oscar_ascend/layout.py:9-95."""

    physical_block_tokens: int
    kv_heads: int = 1
    kernel_block_tokens: int = 128
    config: OscarConfig = field(default_factory=OscarConfig)

    def __post_init__(self):
        # Same accept/reject behaviour as layout.py:15-28.
        if min(self.kv_heads, self.physical_block_tokens) <= 0:
            raise ValueError("physical block tokens and kv heads must be positive")
        if self.physical_block_tokens % self.kernel_block_tokens:
            raise ValueError(
                f"physical block ({self.physical_block_tokens} tokens) is not a multiple of "
                f"the kernel block ({self.kernel_block_tokens} tokens)"
            )
        capacity = self.stripe_page_bytes
        if self.history_page_bytes > capacity:
            raise ValueError("INT2 history slots exceed the native K stripe of a page")
        if self.window_page_bytes > capacity:
            raise ValueError(
                f"the BF16 sink/ring window needs {self.window_page_bytes} bytes per owner "
                f"page but a V stripe page has {capacity}; use a physical block of at least "
                f"{2 * self.config.window_tokens} tokens"
            )

    # ---- sizes (layout.py:30-44)
    @property
    def stripe_page_bytes(self):
        return self.physical_block_tokens * self.kv_heads * self.config.head_dim * 2

    @property
    def history_page_bytes(self):
        return self.physical_block_tokens * self.kv_heads * self.config.slot_bytes

    @property
    def window_page_bytes(self):
        cfg = self.config
        return cfg.window_tokens * 2 * self.kv_heads * cfg.head_dim * 2

    @property
    def blocks_per_page(self):
        return self.physical_block_tokens // self.kernel_block_tokens

    # ---- addressing (layout.py:46-73)
    def slot_offset(self, slot, head=0):
        """Byte offset of a token-head's 160-byte slot in the K stripe."""
        if slot < 0 or head < 0 or head >= self.kv_heads:
            raise ValueError("slot must be >= 0 and head inside [0, kv_heads)")
        page = slot // self.physical_block_tokens
        within = slot - page * self.physical_block_tokens
        return page * self.stripe_page_bytes + (within * self.kv_heads + head) * (
            self.config.slot_bytes
        )

    def logical_slot(self, block_table, position):
        """Physical slot of logical token ``position`` through a 128-token block table row."""
        kernel_block = self.kernel_block_tokens
        return block_table[position // kernel_block] * kernel_block + position % kernel_block

    def window_index(self, position):
        sink = self.config.sink_tokens
        return position if position < sink else sink + position % self.config.ring_tokens

    def window_offset(self, first_kernel_block, position, kv=0, head=0):
        """Byte offset of a window entry (kv=0 K, kv=1 V) in the V stripe."""
        if position < 0 or kv not in (0, 1) or head < 0 or head >= self.kv_heads:
            raise ValueError("invalid window position, kv selector or head")
        if first_kernel_block < 0 or first_kernel_block % self.blocks_per_page:
            raise ValueError("a request's first kernel block must start a physical page")
        owner = first_kernel_block // self.blocks_per_page
        entry = (self.window_index(position) * 2 + kv) * self.kv_heads + head
        return owner * self.stripe_page_bytes + entry * self.config.head_dim * 2

    # ---- views over the native cache (layout.py:75-95)
    def tensor_views(self, kv_cache):
        """(uint8 flat K stripe, bf16 flat V stripe) views of native BF16 K/V caches."""
        import torch

        if not isinstance(kv_cache, (tuple, list)) or len(kv_cache) != 2:
            raise ValueError("expected the native (K, V) cache view pair")
        k, v = kv_cache
        expected = (self.kernel_block_tokens, self.kv_heads, self.config.head_dim)
        for tensor in (k, v):
            if tensor.dtype != torch.bfloat16 or not tensor.is_contiguous():
                raise ValueError("OSCAR needs contiguous BF16 K/V cache views")
            if tensor.ndim != 4 or tuple(tensor.shape[1:]) != expected:
                raise ValueError(f"unexpected native cache shape {tuple(tensor.shape)}")
            if (tensor.numel() * tensor.element_size()) % self.stripe_page_bytes:
                raise ValueError("a native stripe must hold a whole number of physical pages")
        if k.shape != v.shape:
            raise ValueError("K and V stripes must have the same geometry")
        return k.view(torch.uint8).view(-1), v.view(-1)
