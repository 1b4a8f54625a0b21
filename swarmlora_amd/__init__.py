"""swarmlora_amd — MI355X (gfx950) implementation of SwarmLoRA's per-layer
gather -> base-GEMM -> scatter rounds, the LoRA delta and the paged-KV decode
attention, behind the reference's Python-facing APIs.

Python-facing modules (same names and signatures as the reference's pybind
extensions and worker classes):
  swarmlora_amd.ext_aggregator, swarmlora_amd.ext_ipc_queue,
  swarmlora_amd.ext_unified_barrier, swarmlora_amd.worker.*
Kernels: swarmlora_amd.ops (torch tensors) over libswl.so (include/swl.h).
"""

import os

__version__ = "0.1.0"

PKG_DIR = os.path.dirname(os.path.abspath(__file__))


def compat_path():
    """Directory that makes `import ext_aggregator` / `ext_ipc_queue` /
    `ext_unified_barrier` resolve to this package's modules (prepend it to
    sys.path or PYTHONPATH in place of the reference's built extensions)."""
    return os.path.join(PKG_DIR, "compat")
