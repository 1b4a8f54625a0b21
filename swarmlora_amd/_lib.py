"""ctypes binding of libswl.so (the C ABI declared in include/swl.h and
include/swl_runtime.h).

torch is imported before the library is loaded so that the process has one
HIP runtime: libswl.so's NEEDED libamdhip64.so.7 then resolves to the copy
torch already mapped.  The library is built in-tree by swarmlora_amd.build;
nothing here falls back to another implementation when it is missing.
"""

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading libswl.so)

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libswl.so")

_lock = threading.Lock()
_lib = None

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_u64 = ctypes.c_uint64
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p
c_int = ctypes.c_int
P_i64 = ctypes.POINTER(ctypes.c_int64)
P_i32 = ctypes.POINTER(ctypes.c_int32)
P_vp = ctypes.POINTER(ctypes.c_void_p)
P_size = ctypes.POINTER(ctypes.c_size_t)

SWL_MAX_LORA_BLOCKS = 4
# SWL_ABI_VERSION of include/swl.h that the structures and signatures below
# mirror; load() refuses a library built from another version
ABI_VERSION = 2


class LoraEntry(ctypes.Structure):
    """Mirror of swl_lora_entry (include/swl.h)."""
    _fields_ = [
        ("a", c_vp),
        ("b", c_vp * SWL_MAX_LORA_BLOCKS),
        ("rank", c_i32),
        ("scale", c_f32),
    ]


class RoundFusion(ctypes.Structure):
    """swl_round_fusion (include/swl.h)."""
    _fields_ = [
        ("norm_weight", c_vp),
        ("eps", c_f32),
        ("ss_in", c_vp),
        ("ss_in_n", ctypes.c_int32),
        ("ss_in_stride", ctypes.c_int32),
        ("out_mode", ctypes.c_int32),
        ("ss_out", c_vp),
        ("ss_out_stride", ctypes.c_int32),
        ("k_cache", c_vp),
        ("v_cache", c_vp),
        ("hq", ctypes.c_int32),
        ("hkv", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("block_table", c_vp),
        ("max_blocks", c_i64),
        ("num_blocks", c_i64),
        ("cache_seqlens", c_vp),
        ("positions", c_vp),
        ("cos_sin", c_vp),
        ("max_pos", c_i64),
        ("w_layout", ctypes.c_int32),
        ("a_layout", ctypes.c_int32),
    ]


class PoolStatus(ctypes.Structure):
    """Mirror of swl_pool_status (include/swl_runtime.h)."""
    _fields_ = [
        ("initialized", c_i32),
        ("num_slots", c_i32),
        ("free_lo", c_u64),
        ("free_hi", c_u64),
        ("active_lo", c_u64),
        ("active_hi", c_u64),
        ("active_slot_count", c_i32),
        ("owners", c_i32 * 128),
    ]


_SIGS = {
    # kernels (include/swl.h)
    "swl_last_error": (ctypes.c_char_p, []),
    "swl_abi_version": (c_int, []),
    "swl_device_count": (c_int, []),
    "swl_gather_bf16": (c_int, [P_vp, P_i64, c_int, c_i64, c_vp, c_vp]),
    "swl_scatter_add_bf16": (c_int, [c_vp, c_vp, P_vp, P_i64, c_int, c_i64, c_vp]),
    "swl_gemm_bf16": (c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp]),
    "swl_round_bf16": (c_int, [c_int, P_i64, P_vp, P_vp, c_vp, c_vp, c_i64, c_i64, P_i32, c_vp, c_vp, c_int,
                               P_i64, c_vp]),
    "swl_round_ex_bf16": (c_int, [c_int, P_i64, P_vp, P_vp, c_vp, c_vp, c_i64, c_i64, P_i32, c_vp, c_vp, c_int,
                                  P_i64, ctypes.POINTER(RoundFusion), c_vp]),
    "swl_round_ex_noalloc_bf16": (c_int, [c_int, P_i64, P_vp, P_vp, c_vp, c_vp, c_i64, c_i64, P_i32, c_vp, c_vp, c_int,
                                  P_i64, ctypes.POINTER(RoundFusion), c_vp]),
    "swl_pack_weight_bf16": (c_int, [c_vp, c_i64, c_i64, c_vp, c_vp]),
    "swl_lora_segmented_bf16": (c_int, [c_vp, c_i64, c_int, P_i64, P_i32, c_vp, c_vp, c_int, P_i64, c_vp, c_i64,
                                        c_int, c_vp]),
    "swl_matmul_bf16": (c_int, [c_vp, c_i64, c_vp, c_i64, c_int, c_vp, c_i64, c_i64, c_i64, c_i64, c_f32,
                                c_vp]),
    "swl_lora_rows_bf16": (c_int, [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_int, c_i64, P_vp, P_i64,
                                   P_i64, P_i64, c_f32, c_vp, c_i64, c_vp]),
    "swl_paged_attention_bf16": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_int, c_int,
                                         c_vp, c_vp, c_i64, c_int, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int,
                                         c_f32, c_vp, c_vp]),
    "swl_embed_bf16": (c_int, [P_vp, P_i64, c_int, c_vp, c_i64, c_i64, P_vp, c_vp]),
    "swl_sample_bf16": (c_int, [c_vp, c_i64, c_i64, P_vp, P_i32, ctypes.POINTER(c_f32), P_i32,
                                ctypes.POINTER(c_f32), c_u64, c_vp]),
    "swl_zero_blocks_bf16": (c_int, [P_vp, c_int, c_vp, c_i64, c_i64, c_vp]),
    "swl_timer_arm": (c_int, [c_int]),
    "swl_timer_collect": (c_int, [c_int, ctypes.POINTER(c_f32), ctypes.POINTER(c_f32), P_i64, P_i64, P_i32, P_i64,
                                  ctypes.POINTER(c_int)]),
    "swl_rmsnorm_rows_bf16": (c_int, [c_vp, c_i64, c_i64, P_vp, c_vp, c_f32, P_vp, c_vp]),
    "swl_silu_mul_rows_bf16": (c_int, [P_vp, P_vp, c_i64, c_i64, c_vp]),
    "swl_paged_attention_rows_bf16": (c_int, [P_vp, P_vp, c_int, c_int, c_int, c_int, c_int, c_vp, c_vp, c_i64,
                                              c_int, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_f32, c_vp]),
}

_RUNTIME_SIGS = {}


def register_signatures(sigs):
    """Runtime modules add their entry points before the first load()."""
    _RUNTIME_SIGS.update(sigs)
    if _lib is not None:
        _declare(_lib, sigs)


def _declare(lib, sigs):
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load():
    """Load libswl.so once (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m swarmlora_amd.build` "
                    "(the HIP path has no fallback)")
            lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
            lib.swl_abi_version.restype = c_int
            got = lib.swl_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI version {got}, this binding expects {ABI_VERSION}: "
                                   "rebuild it with `python -m swarmlora_amd.build`")
            _declare(lib, _SIGS)
            _declare(lib, _RUNTIME_SIGS)
            _lib = lib
    return _lib


def last_error():
    msg = load().swl_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc):
    """Raise RuntimeError with the library's message on a non-zero status."""
    if rc != 0:
        raise RuntimeError(last_error() or f"libswl error {rc}")
    return rc


def exported_symbols():
    """Names of every entry point the Python side declares."""
    return sorted(list(_SIGS) + list(_RUNTIME_SIGS))
