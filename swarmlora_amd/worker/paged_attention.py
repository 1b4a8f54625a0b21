"""Paged KV cache block manager and the RoPE cos/sin cache.

Same class, constructor and methods as the reference's
src/worker/paged_attention.py (PagedKVCache :7-128,
build_vllm_cos_sin_cache :131-142).  Pages use the flash-attn layout
[num_blocks, block_size, num_kv_heads, head_dim] the libswl attention kernel
reads; freed pages are zeroed by a libswl kernel.
"""

import math
from typing import Dict, List, Optional

import torch

from .. import ops


class PagedKVCache:
    """Per-layer K and V page pools with a LIFO free list (the first
    allocations get blocks 0, 1, 2, ...), per-slot block tables and
    sequence lengths."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, block_size: int, max_slots: int,
                 max_seq_len: int, device, dtype: torch.dtype):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.device = device
        self.dtype = dtype
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        self.num_blocks = max_slots * self.max_blocks_per_seq
        shape = (self.num_blocks, block_size, num_kv_heads, head_dim)
        self.key_caches = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(num_layers)]
        self.value_caches = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(num_layers)]
        self.free_blocks = list(range(self.num_blocks - 1, -1, -1))
        self.slot_block_tables: Dict[int, List[int]] = {}
        self.slot_seq_lens: Dict[int, int] = {}

    def allocate_blocks(self, slot_id: int, num_blocks: int):
        if len(self.free_blocks) < num_blocks:
            raise RuntimeError(f"PagedKVCache: need {num_blocks} blocks but only {len(self.free_blocks)} free")
        blocks = [self.free_blocks.pop() for _ in range(num_blocks)]
        if slot_id in self.slot_block_tables:
            self.slot_block_tables[slot_id].extend(blocks)
        else:
            self.slot_block_tables[slot_id] = blocks
            self.slot_seq_lens[slot_id] = 0

    def ensure_blocks_for_length(self, slot_id: int, needed_len: int):
        needed = (needed_len + self.block_size - 1) // self.block_size
        if needed > self.max_blocks_per_seq:
            raise RuntimeError(f"PagedKVCache: {needed_len} tokens exceed max_seq_len")
        current = len(self.slot_block_tables.get(slot_id, []))
        if needed > current:
            self.allocate_blocks(slot_id, needed - current)

    def free_slot(self, slot_id: int):
        """Return the slot's blocks to the free list after zeroing them in every
        layer (no KV leaks across requests)."""
        blocks = self.slot_block_tables.pop(slot_id, [])
        if blocks:
            assert all(0 <= b < self.num_blocks for b in blocks)
            ids = torch.tensor(blocks, dtype=torch.int64, device=self.device)
            ops.zero_blocks(self.key_caches + self.value_caches, ids)
        self.free_blocks.extend(blocks)
        self.slot_seq_lens.pop(slot_id, None)

    def get_block_table_tensor(self, slot_ids: List[int]) -> torch.Tensor:
        """int32 [len(slot_ids), max_blocks_per_seq], zero-padded (a new tensor)."""
        bt = torch.zeros(len(slot_ids), self.max_blocks_per_seq, dtype=torch.int32)
        for i, sid in enumerate(slot_ids):
            blocks = self.slot_block_tables[sid]
            bt[i, :len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
        return bt.to(self.device)

    def get_seq_lens_tensor(self, slot_ids: List[int]) -> torch.Tensor:
        """int32 [len(slot_ids)] (a new tensor)."""
        return torch.tensor([self.slot_seq_lens[s] for s in slot_ids], dtype=torch.int32).to(self.device)

    def advance_seq_lens(self, slot_ids: List[int], count: int = 1):
        for sid in slot_ids:
            self.slot_seq_lens[sid] += count

    def advance_seq_lens_by(self, slot_ids: List[int], counts: List[int]):
        for sid, c in zip(slot_ids, counts):
            self.slot_seq_lens[sid] += c


def build_vllm_cos_sin_cache(rotary_emb, max_seq_len: int, device, dtype: torch.dtype) -> torch.Tensor:
    """[max_seq_len, head_dim] = cat(cos, sin) of outer(arange fp32, inv_freq),
    cast to `dtype` (paged_attention.py:131-142).  `rotary_emb` is anything
    with an `inv_freq` tensor (HF LlamaRotaryEmbedding)."""
    t = torch.arange(max_seq_len, device=device, dtype=torch.float32)
    inv_freq = rotary_emb.inv_freq.to(device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat([freqs.cos().to(dtype), freqs.sin().to(dtype)], dim=-1).contiguous()


class RotaryInvFreq:
    """Stand-in for HF LlamaRotaryEmbedding's `inv_freq` (the rotary that
    model_builder.py:293-296 builds from the model config): theta^(-2i/d),
    and with rope_scaling of type "llama3" (Llama 3.1 configs) the Llama 3.1
    frequency remap: f / factor for wavelengths above
    original_max_position_embeddings / low_freq_factor, f below
    original_max_position_embeddings / high_freq_factor, a linear blend in
    between."""

    def __init__(self, head_dim: int, theta: float, device="cpu", rope_scaling: Optional[dict] = None):
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64, device=device).float() / head_dim))
        kind = (rope_scaling or {}).get("rope_type", (rope_scaling or {}).get("type", "default"))
        if kind == "llama3":
            factor = float(rope_scaling["factor"])
            lo = float(rope_scaling["low_freq_factor"])
            hi = float(rope_scaling["high_freq_factor"])
            old_len = float(rope_scaling["original_max_position_embeddings"])
            wavelen = 2 * math.pi / inv
            scaled = torch.where(wavelen > old_len / lo, inv / factor, inv)
            smooth = (old_len / wavelen - lo) / (hi - lo)
            blended = (1 - smooth) * scaled / factor + smooth * scaled
            medium = (wavelen >= old_len / hi) & (wavelen <= old_len / lo)
            inv = torch.where(medium, blended, scaled)
        elif kind != "default":
            raise ValueError(f"rope_scaling type {kind!r} is not supported")
        self.inv_freq = inv
