"""Worker-side classes of the hot path (LoRA modules, paged KV cache, round
helpers, per-token driver) on the libswl kernels."""
