"""The C-ABI library loads on a host without a GPU and exports every entry
point declared in include/*.h (no compute calls here)."""

import glob
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^\s*(?:const\s+)?(?:int|int64_t|char|void)\s*\*?\s*(swl_[a-z0-9_]+)\s*\(", re.M)


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        names.update(DECL.findall(open(h).read()))
    return sorted(names)


def test_headers_declare_entry_points():
    assert "swl_round_bf16" in declared_symbols()
    assert len(declared_symbols()) >= 10


def test_library_exports_every_declared_symbol():
    from swarmlora_amd import _lib
    from swarmlora_amd import ext_aggregator, ext_ipc_queue, ext_unified_barrier  # noqa: F401
    lib = _lib.load()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the Python side declares a signature for every header entry point
    assert set(declared_symbols()) <= set(_lib.exported_symbols())


def test_error_text_and_no_device_calls():
    from swarmlora_amd import _lib
    lib = _lib.load()
    assert lib.swl_abi_version() >= 1
    assert lib.swl_device_count() >= 0
    # argument validation fails before any HIP call
    rc = lib.swl_gemm_bf16(None, None, None, None, 1, 1, 32, None)
    assert rc != 0 and "null argument" in _lib.last_error()


def test_slot_pool_refuses_buffers_past_the_ipc_limit():
    """init_slot_pool refuses slot buffers of 2 GiB or more (an IPC mapping
    of that size does not open) before it touches the device."""
    from swarmlora_amd import ext_aggregator as agg
    # 8B shapes: out = max_seq x max(2 x 14336, 6144) x 2 B; 37450 rows -> 2.0 GiB
    with pytest.raises(RuntimeError, match="2 GiB limit of an IPC mapping"):
        agg.init_slot_pool(4, 0, 4096, 14336, 8, 128, 37450, 2)
