"""torch-tensor front end of the libswl kernels.

Every function here validates shapes on the host (the kernels and their grids
assume them), then calls the C ABI on torch's current HIP stream.  There is no
CPU or torch fallback: on a host without the built library or a GPU these
raise.
"""

import ctypes
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import LoraEntry, SWL_MAX_LORA_BLOCKS

BF16 = torch.bfloat16


# The current stream's raw handle.  torch.cuda.current_stream() builds a
# Stream object and checks the device on every call (~2.7 us against ~0.2 us
# here, measured on MI355X); a worker makes a few dozen such calls per round.
if hasattr(torch._C, "_cuda_getCurrentRawStream") and hasattr(torch._C, "_cuda_getDevice"):
    def _stream():
        return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice()))
else:
    def _stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _need(t: torch.Tensor, name: str, dtype=BF16):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the HIP path has no CPU fallback)")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def _ptr_array(ts: Sequence[Optional[torch.Tensor]]):
    arr = (ctypes.c_void_p * len(ts))()
    for i, t in enumerate(ts):
        arr[i] = t.data_ptr() if t is not None else 0
    return arr


def _i64_array(vals):
    arr = (ctypes.c_int64 * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr


def _i32_array(vals):
    arr = (ctypes.c_int32 * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr


def gather(slot_inputs: Sequence[torch.Tensor], rows: Sequence[int], out: Optional[torch.Tensor] = None):
    """Pack rows[i] leading rows of each slot buffer (2-D [>= rows[i], d]) into
    one [sum(rows), d] tensor, in the given order."""
    d = slot_inputs[0].shape[-1]
    for i, t in enumerate(slot_inputs):
        _need(t, f"slot_inputs[{i}]")
        if t.shape[-1] != d or not t.is_contiguous() or t.numel() < rows[i] * d:
            raise ValueError("slot inputs must be contiguous [rows, d] with a common d")
    total = int(sum(rows))
    if out is None:
        out = torch.empty(total, d, dtype=BF16, device=slot_inputs[0].device)
    _lib.check(_lib.load().swl_gather_bf16(_ptr_array(slot_inputs), _i64_array(rows), len(rows), d,
                                           _ptr(out), _stream()))
    return out


def scatter_add(y: torch.Tensor, slot_outputs: Sequence[torch.Tensor], rows: Sequence[int],
                delta: Optional[torch.Tensor] = None):
    """slot_outputs[i][:rows[i]] = y[off_i : off_i + rows[i]] (+ delta ...)."""
    _need(y, "y")
    d = y.shape[-1]
    if delta is not None:
        _need(delta, "delta")
        if delta.shape != y.shape:
            raise ValueError("delta must match y")
    for i, t in enumerate(slot_outputs):
        _need(t, f"slot_outputs[{i}]")
        if not t.is_contiguous() or t.numel() < rows[i] * d:
            raise ValueError("slot outputs must be contiguous and hold rows[i] * d elements")
    if y.shape[0] != sum(rows):
        raise ValueError("y rows must equal sum(rows)")
    _lib.check(_lib.load().swl_scatter_add_bf16(_ptr(y.contiguous()), _ptr(delta), _ptr_array(slot_outputs),
                                                _i64_array(rows), len(rows), d, _stream()))


def gemm(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None,
         out: Optional[torch.Tensor] = None):
    """y = x @ w.T (+ bias), bf16 in/out, fp32 accumulate."""
    _need(x, "x")
    _need(w, "w")
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError("gemm expects x [m, k] and w [n, k]")
    if not (x.is_contiguous() and w.is_contiguous()):
        raise ValueError("gemm operands must be contiguous")
    m, k = x.shape
    n = w.shape[0]
    if bias is not None:
        _need(bias, "bias")
        if bias.numel() != n:
            raise ValueError("bias must have n elements")
    if out is None:
        out = torch.empty(m, n, dtype=BF16, device=x.device)
    _lib.check(_lib.load().swl_gemm_bf16(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), m, n, k, _stream()))
    return out


class LoraTable:
    """Device array of swl_lora_entry records.  Keeps the tensors it points to
    alive.  Entry i describes one adapter for one (fused) projection."""

    def __init__(self, device):
        self.device = torch.device(device)
        self._entries: List[LoraEntry] = []
        self._packed: List[bool] = []
        self._keep = []
        self._dev = None

    def add(self, a, bs: Sequence[torch.Tensor], rank: int, scale: float) -> int:
        """a: bf16 [nblk*rank, k] (stacked lora_A), or its PackedWeight
        (fragment tiles: the K-sliced decode rounds stream it like the
        weights, round fusion a_layout 1); bs[j]: bf16 [blk_cols[j], rank]."""
        packed = isinstance(a, PackedWeight)
        if packed:
            if a.n != rank * len(bs):
                raise ValueError("packed lora a must be a PackedWeight of [nblk * rank, k]")
        else:
            _need(a, "lora a")
            if not a.is_contiguous() or a.shape[0] != rank * len(bs):
                raise ValueError("lora a must be contiguous [nblk * rank, k]")
        if len(bs) > SWL_MAX_LORA_BLOCKS:
            raise ValueError("too many column blocks")
        e = LoraEntry()
        e.a = a.data_ptr()
        for j, b in enumerate(bs):
            _need(b, f"lora b[{j}]")
            if not b.is_contiguous() or b.shape[1] != rank:
                raise ValueError("lora b must be contiguous [cols, rank]")
            e.b[j] = b.data_ptr()
        e.rank = int(rank)
        e.scale = float(scale)
        self._entries.append(e)
        self._packed.append(packed)
        self._keep.extend([a, *bs])
        self._dev = None
        return len(self._entries) - 1

    def a_layout(self, ids: Sequence[int]) -> int:
        """Layout of lora_A over the entries `ids` (negative: none): 1 if
        they are fragment tiles, 0 if row-major; mixed layouts are refused
        (a round streams one kind)."""
        kinds = {self._packed[i] for i in ids if i >= 0}
        if len(kinds) > 1:
            raise ValueError("a round's adapters must all have row-major or all fragment-tile lora_A")
        return 1 if kinds == {True} else 0

    def _sync(self):
        if self._dev is None:
            n = len(self._entries)
            self._host = (LoraEntry * max(n, 1))(*self._entries)
            host = torch.frombuffer(bytearray(bytes(self._host)), dtype=torch.uint8)
            self._dev = host.to(self.device)

    def device_table(self) -> torch.Tensor:
        self._sync()
        return self._dev

    def host_table(self):
        """ctypes array of the same records (host memory)."""
        self._sync()
        return self._host

    def __len__(self):
        return len(self._entries)


class PackedWeight:
    """Fragment-tile copy of a row-major weight [n, k] for decode-shaped
    rounds (swl_pack_weight_bf16): 16-row tiles stored whole, k-step by
    k-step, each k-step block the MFMA A operand of those rows.  `data` is
    flat bf16 of ceil(n / 16) * 16 * k elements."""

    def __init__(self, w: torch.Tensor):
        _need(w, "w")
        if w.dim() != 2 or not w.is_contiguous():
            raise ValueError("w must be a contiguous [n, k] matrix")
        self.n, self.k = w.shape
        if self.k % 32:
            raise ValueError("k must be a multiple of 32")
        self.data = torch.empty((self.n + 15) // 16 * 16 * self.k, dtype=BF16, device=w.device)
        _lib.check(_lib.load().swl_pack_weight_bf16(_ptr(w), self.n, self.k, _ptr(self.data), _stream()))

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.data.device

    def data_ptr(self):
        return self.data.data_ptr()


def pack_weight(w: torch.Tensor) -> PackedWeight:
    """Fragment-tile copy of w [n, k] (see PackedWeight)."""
    return PackedWeight(w)


def _round_args(seg_in, seg_out, rows, w, bias, seg_lora, table, blk_cols, out_div=1):
    if not isinstance(w, PackedWeight):
        _need(w, "w")
    n, k = w.shape
    if len(seg_in) != len(rows) or len(seg_out) != len(rows):
        raise ValueError("one input, output and row count per segment")
    for i in range(len(rows)):
        _need(seg_in[i], f"seg_in[{i}]")
        _need(seg_out[i], f"seg_out[{i}]")
        if seg_in[i].numel() < rows[i] * k or seg_out[i].numel() < rows[i] * (n // out_div):
            raise ValueError(f"segment {i} buffers are smaller than rows * dim")
        if not (seg_in[i].is_contiguous() and seg_out[i].is_contiguous()):
            raise ValueError("segment buffers must be contiguous")
    if bias is not None:
        _need(bias, "bias")
    lora_arr = None
    tab_ptr = ctypes.c_void_p(0)
    host_tab = ctypes.c_void_p(0)
    blk = None
    nblk = 0
    if seg_lora is not None:
        if table is None or blk_cols is None:
            raise ValueError("seg_lora needs a LoraTable and blk_cols")
        if any(i >= len(table) for i in seg_lora):
            raise ValueError("seg_lora index out of range")
        lora_arr = _i32_array(seg_lora)
        tab_ptr = _ptr(table.device_table())
        host_tab = ctypes.cast(table.host_table(), ctypes.c_void_p)
        blk = _i64_array(blk_cols)
        nblk = len(blk_cols)
    return (len(rows), _i64_array(rows), _ptr_array(seg_in), _ptr_array(seg_out), _ptr(w), _ptr(bias), n, k,
            lora_arr, tab_ptr, host_tab, nblk, blk)


def round_fused(seg_in: Sequence[torch.Tensor], seg_out: Sequence[torch.Tensor], rows: Sequence[int],
                w: torch.Tensor, bias: Optional[torch.Tensor] = None,
                seg_lora: Optional[Sequence[int]] = None, table: Optional[LoraTable] = None,
                blk_cols: Optional[Sequence[int]] = None):
    """One gather -> GEMM -> (+LoRA) -> scatter round over slot buffers."""
    if isinstance(w, PackedWeight) or (seg_lora is not None and table is not None and table.a_layout(seg_lora)):
        return round_ex(seg_in, seg_out, rows, w, bias, seg_lora, table, blk_cols)
    args = _round_args(seg_in, seg_out, rows, w, bias, seg_lora, table, blk_cols)
    _lib.check(_lib.load().swl_round_bf16(*args, _stream()))


RoundFusion = _lib.RoundFusion


def round_fusion(norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-5,
                 ss_in: Optional[torch.Tensor] = None, out_mode: int = 0, ss_out: Optional[torch.Tensor] = None,
                 k_cache: Optional[torch.Tensor] = None, v_cache: Optional[torch.Tensor] = None, hq: int = 0,
                 hkv: int = 0, block_table: Optional[torch.Tensor] = None,
                 cache_seqlens: Optional[torch.Tensor] = None, positions: Optional[torch.Tensor] = None,
                 cos_sin: Optional[torch.Tensor] = None, w_layout: int = 0, a_layout: int = 0) -> RoundFusion:
    """swl_round_fusion for round_ex (include/swl.h documents each mode).
    ss_in / ss_out: fp32 [ntok, n_partial] (n_partial = ceil(n / 256) of the
    producing round); the record keeps the tensors it points to alive."""
    f = RoundFusion()
    keep = []
    if w_layout not in (0, 1, 2):
        raise ValueError("w_layout must be 0 (row-major), 1 (fragment tiles) or 2 (whole-K round)")
    f.w_layout = w_layout
    if a_layout not in (0, 1) or (a_layout == 1 and w_layout == 2):
        raise ValueError("a_layout must be 0 (row-major lora_A) or 1 (fragment tiles, w_layout 0 or 1)")
    f.a_layout = a_layout
    if norm_weight is not None:
        _need(norm_weight, "norm_weight")
        _need(ss_in, "ss_in", torch.float32)
        if ss_in.dim() != 2 or ss_in.stride(1) != 1:
            raise ValueError("ss_in must be [ntok, n_partial] with unit column stride")
        f.norm_weight, f.eps = norm_weight.data_ptr(), float(eps)
        f.ss_in, f.ss_in_n, f.ss_in_stride = ss_in.data_ptr(), ss_in.shape[1], ss_in.stride(0)
        keep += [norm_weight, ss_in]
    if out_mode not in (0, 1, 2, 3):
        raise ValueError("out_mode must be 0..3")
    f.out_mode = out_mode
    if out_mode == 1:
        _need(ss_out, "ss_out", torch.float32)
        if ss_out.dim() != 2 or ss_out.stride(1) != 1:
            raise ValueError("ss_out must be [ntok, n_partial] with unit column stride")
        f.ss_out, f.ss_out_stride = ss_out.data_ptr(), ss_out.stride(0)
        keep.append(ss_out)
    if out_mode == 3:
        for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
            _need(t, nm)
            if not t.is_contiguous() or t.dim() != 4 or t.shape[2] != hkv or t.shape[3] != 128:
                raise ValueError(f"{nm} must be contiguous [num_blocks, block_size, hkv, 128]")
        _need(block_table, "block_table", torch.int32)
        _need(cache_seqlens, "cache_seqlens", torch.int32)
        _need(positions, "positions", torch.int64)
        _need(cos_sin, "cos_sin")
        if block_table.dim() != 2 or not block_table.is_contiguous():
            raise ValueError("block_table must be contiguous [nseq, max_blocks]")
        if cos_sin.dim() != 2 or cos_sin.shape[1] != 128 or not cos_sin.is_contiguous():
            raise ValueError("cos_sin must be contiguous [max_pos, 128]")
        f.k_cache, f.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
        f.hq, f.hkv, f.block_size = hq, hkv, k_cache.shape[1]
        f.block_table, f.max_blocks, f.num_blocks = block_table.data_ptr(), block_table.shape[1], k_cache.shape[0]
        f.cache_seqlens, f.positions = cache_seqlens.data_ptr(), positions.data_ptr()
        f.cos_sin, f.max_pos = cos_sin.data_ptr(), cos_sin.shape[0]
        keep += [k_cache, v_cache, block_table, cache_seqlens, positions, cos_sin]
    f._keep = keep
    return f


def round_ex(seg_in: Sequence[torch.Tensor], seg_out: Sequence[torch.Tensor], rows: Sequence[int],
             w: torch.Tensor, bias: Optional[torch.Tensor] = None,
             seg_lora: Optional[Sequence[int]] = None, table: Optional[LoraTable] = None,
             blk_cols: Optional[Sequence[int]] = None, fusion: Optional[RoundFusion] = None,
             noalloc: bool = False):
    """round_fused with the decode-step fusions of `fusion` (round_fusion()).
    A PackedWeight w runs the K-sliced decode round (w_layout 1) unless the
    fusion asks for the whole-K round (w_layout 2: out_mode 0 only, the
    decode step's LM head).
    noalloc=True calls the allocation-free entry point
    (swl_round_ex_noalloc_bf16: at most 64 token rows, partials in the
    library's fixed 64 MiB device array)."""
    if isinstance(w, PackedWeight):
        if fusion is None:
            fusion = RoundFusion()
        if fusion.w_layout != 2:
            fusion.w_layout = 1
        elif fusion.out_mode != 0:
            raise ValueError("the whole-K round (w_layout 2) has out_mode 0 only")
    elif fusion is not None and fusion.w_layout != 0:
        raise ValueError("fusion.w_layout 1 or 2 needs a PackedWeight")
    if seg_lora is not None and table is not None and table.a_layout(seg_lora) == 1:
        if fusion is None:
            fusion = RoundFusion()
        if fusion.w_layout == 2:
            raise ValueError("fragment-tile lora_A needs a K-sliced round (w_layout 0 or 1)")
        fusion.a_layout = 1
    elif fusion is not None and fusion.a_layout != 0:
        raise ValueError("fusion.a_layout 1 needs adapters added with a PackedWeight lora_A")
    args = _round_args(seg_in, seg_out, rows, w, bias, seg_lora, table, blk_cols,
                       out_div=2 if fusion is not None and fusion.out_mode == 2 else 1)
    fn = _lib.load().swl_round_ex_noalloc_bf16 if noalloc else _lib.load().swl_round_ex_bf16
    _lib.check(fn(*args, ctypes.byref(fusion) if fusion is not None else None, _stream()))


def lora_segmented(x: torch.Tensor, seg_rows: Sequence[int], seg_lora: Sequence[int], table: LoraTable,
                   blk_cols: Sequence[int], y: torch.Tensor, add: bool = False):
    """Segmented LoRA delta of the packed rows x [T, k] (swl_lora_segmented_bf16):
    y [T, n] = delta (add=False) or y += delta (add=True); segment i's rows use
    table entry seg_lora[i] (-1: no adapter)."""
    _need(x, "x")
    _need(y, "y")
    if x.dim() != 2 or not x.is_contiguous() or y.dim() != 2 or not y.is_contiguous():
        raise ValueError("x and y must be contiguous 2-D tensors")
    if len(seg_rows) != len(seg_lora):
        raise ValueError("one adapter index per segment")
    t = sum(int(r) for r in seg_rows)
    if x.shape[0] != t or y.shape[0] != t:
        raise ValueError("x and y need sum(seg_rows) rows")
    if any(i >= len(table) for i in seg_lora):
        raise ValueError("seg_lora index out of range")
    if table.a_layout(seg_lora):
        raise ValueError("the segmented LoRA delta reads row-major lora_A")
    _lib.check(_lib.load().swl_lora_segmented_bf16(
        _ptr(x), x.shape[1], len(seg_rows), _i64_array(seg_rows), _i32_array(seg_lora), _ptr(table.device_table()),
        ctypes.cast(table.host_table(), ctypes.c_void_p), len(blk_cols), _i64_array(blk_cols), _ptr(y), y.shape[1],
        1 if add else 0, _stream()))
    return y


def matmul(x: torch.Tensor, b: torch.Tensor, trans_b: bool, alpha: float = 1.0,
           out: Optional[torch.Tensor] = None):
    """y = alpha * x @ (b.T if trans_b else b) for 2-D views with unit column
    stride (row strides may be arbitrary).  fp32 accumulation, bf16 output."""
    _need(x, "x")
    _need(b, "b")
    if x.dim() != 2 or b.dim() != 2:
        raise ValueError("matmul expects 2-D operands")
    if x.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("matmul operands need unit column stride")
    m, k = x.shape
    n = b.shape[0] if trans_b else b.shape[1]
    kb = b.shape[1] if trans_b else b.shape[0]
    if kb != k:
        raise ValueError("matmul inner dimensions differ")
    if out is None:
        out = torch.empty(m, n, dtype=BF16, device=x.device)
    if out.stride(1) != 1:
        raise ValueError("out needs unit column stride")
    _lib.check(_lib.load().swl_matmul_bf16(_ptr(x), x.stride(0), _ptr(b), b.stride(0), 1 if trans_b else 0,
                                           _ptr(out), out.stride(0), m, n, k, float(alpha), _stream()))
    return out


LORA_ROWS_MAX = 4      # token rows of one lora_rows launch
LORA_ROWS_MAX_NR = 64  # shrink columns (blocks x rank)


def lora_rows(x: torch.Tensor, a: torch.Tensor, a_kmajor: bool, blocks: list, rank: int, alpha: float = 1.0,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """A worker's LoRA delta in one launch (swl_lora_rows_bf16):
    u = bf16(x @ A) with A = a ([k, nr], a_kmajor) or a.T (a is [nr, k]),
    then per column block (b, cols, rr_major): bf16(alpha * u[:, blk*rank:
    (blk+1)*rank] @ B) where B is b [rank, cols] (rr_major, e.g. a diagonal
    block of fused_B) or b.T (b is [cols, rank], e.g. lora_B).  x is [m, k]
    with m <= LORA_ROWS_MAX; returns [m, sum(cols)]."""
    _need(x, "x")
    _need(a, "a")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("lora_rows: x must be 2-D with unit column stride")
    m, k = x.shape
    nr = a.shape[1] if a_kmajor else a.shape[0]
    if (a.shape[0] if a_kmajor else a.shape[1]) != k:
        raise ValueError("lora_rows: A does not match x")
    n = len(blocks)
    ptrs = (ctypes.c_void_p * n)()
    srr = (ctypes.c_int64 * n)()
    sc = (ctypes.c_int64 * n)()
    cols = (ctypes.c_int64 * n)()
    for i, (b, c, rr_major) in enumerate(blocks):
        _need(b, "b")
        ptrs[i] = b.data_ptr()
        if rr_major:
            srr[i], sc[i] = b.stride(0), b.stride(1)
        else:
            srr[i], sc[i] = b.stride(1), b.stride(0)
        cols[i] = int(c)
    total = int(sum(int(c) for _, c, _ in blocks))
    if out is None:
        out = torch.empty(m, total, dtype=BF16, device=x.device)
    _lib.check(_lib.load().swl_lora_rows_bf16(
        _ptr(x), x.stride(0), m, k, _ptr(a), a.stride(0) if a_kmajor else a.stride(1),
        a.stride(1) if a_kmajor else a.stride(0), nr, n, int(rank), ptrs, srr, sc, cols, float(alpha), _ptr(out),
        out.stride(0), _stream()))
    return out


def _token_rows(t: torch.Tensor, name: str, heads: int, d: int):
    """t is [nseq, L, heads, d] whose heads/dims are contiguous per token and
    whose tokens (nseq*L of them) are evenly strided: returns the stride."""
    if t.dim() != 4 or t.shape[2] != heads or t.shape[3] != d:
        raise ValueError(f"{name} must be [nseq, q_len, {heads}, {d}]")
    if t.stride(3) != 1 or t.stride(2) != d:
        raise ValueError(f"{name} heads must be contiguous within a token")
    nseq, L = t.shape[0], t.shape[1]
    if L > 1 and nseq > 1 and t.stride(0) != L * t.stride(1):
        raise ValueError(f"{name} tokens must be evenly strided")
    return t.stride(1) if L > 1 else t.stride(0)


def paged_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, block_table: torch.Tensor, cache_seqlens: torch.Tensor,
                    positions: Optional[torch.Tensor], cos_sin: Optional[torch.Tensor],
                    softmax_scale: float, rope: bool = True, out: Optional[torch.Tensor] = None):
    """q [nseq, L, hq, d], k/v [nseq, L, hkv, d] (views into the fused QKV
    output are fine: tokens may be strided), caches [num_blocks, block_size,
    hkv, d], block_table int32 [nseq, max_blocks], cache_seqlens int32 [nseq],
    positions int64 [nseq*L].  q and k are rotated in place when rope.
    Returns out [nseq, L, hq*d]."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, nm)
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    _need(block_table, "block_table", torch.int32)
    _need(cache_seqlens, "cache_seqlens", torch.int32)
    nseq, L, hq, d = q.shape
    hkv = k.shape[2]
    qs = _token_rows(q, "q", hq, d)
    ks = _token_rows(k, "k", hkv, d)
    vs = _token_rows(v, "v", hkv, d)
    if k.shape[:2] != (nseq, L) or v.shape[:2] != (nseq, L):
        raise ValueError("k and v must be [nseq, L, hkv, d]")
    nb, bs, hkv2, d2 = k_cache.shape
    if v_cache.shape != k_cache.shape or hkv2 != hkv or d2 != d:
        raise ValueError("cache geometry mismatch")
    if block_table.dim() != 2 or block_table.shape[0] < nseq or not block_table.is_contiguous():
        raise ValueError("block_table must be contiguous [nseq, max_blocks]")
    if cache_seqlens.numel() < nseq:
        raise ValueError("cache_seqlens must have nseq entries")
    max_pos = 0
    if rope:
        _need(positions, "positions", torch.int64)
        _need(cos_sin, "cos_sin")
        if positions.numel() != nseq * L:
            raise ValueError("positions must have nseq * q_len entries")
        if cos_sin.shape[-1] != d or not cos_sin.is_contiguous():
            raise ValueError("cos_sin must be contiguous [max_pos, d]")
        max_pos = cos_sin.shape[0]
    if out is None:
        out = torch.empty(nseq, L, hq * d, dtype=BF16, device=q.device)
    else:
        _need(out, "out")
        if out.numel() != nseq * L * hq * d or not out.is_contiguous():
            raise ValueError("out must be contiguous [nseq, L, hq * d]")
    _lib.check(_lib.load().swl_paged_attention_bf16(
        _ptr(q), _ptr(k), _ptr(v), qs, ks, vs, nseq, L, hq, hkv, d, _ptr(k_cache), _ptr(v_cache), nb, bs,
        _ptr(block_table), block_table.shape[1], _ptr(cache_seqlens), _ptr(positions if rope else None),
        _ptr(cos_sin if rope else None), max_pos, 1 if rope else 0, float(softmax_scale), _ptr(out), _stream()))
    return out


def embed(ids: Sequence[torch.Tensor], table: torch.Tensor, outs: Sequence[torch.Tensor]):
    """outs[i][j] = table[clamp(ids[i][j])] for int64 id tensors."""
    _need(table, "table")
    vocab, hidden = table.shape
    for i, t in enumerate(ids):
        _need(t, f"ids[{i}]", torch.int64)
        _need(outs[i], f"outs[{i}]")
        if outs[i].numel() < t.numel() * hidden:
            raise ValueError("embedding output too small")
    _lib.check(_lib.load().swl_embed_bf16(_ptr_array(ids), _i64_array([t.numel() for t in ids]), len(ids),
                                          _ptr(table), vocab, hidden, _ptr_array(outs), _stream()))


def sample(logits: torch.Tensor, out_tok: Sequence[torch.Tensor], do_sample: Sequence[bool],
           temperature: Sequence[float], top_k: Sequence[int], top_p: Sequence[float], seed: int = 0):
    """Next token of each logits row into out_tok[i][0] (int64 device tensors)."""
    _need(logits, "logits")
    n, vocab = logits.shape
    if not logits.is_contiguous():
        raise ValueError("logits must be contiguous")
    for i, t in enumerate(out_tok):
        _need(t, f"out_tok[{i}]", torch.int64)
    f32 = lambda xs: (ctypes.c_float * n)(*[float(x) for x in xs])  # noqa: E731
    _lib.check(_lib.load().swl_sample_bf16(_ptr(logits), n, vocab, _ptr_array(out_tok),
                                           _i32_array([1 if d else 0 for d in do_sample]), f32(temperature),
                                           _i32_array(top_k), f32(top_p), int(seed), _stream()))


def zero_blocks(caches: Sequence[torch.Tensor], block_ids: torch.Tensor):
    """Zero whole pages block_ids of every cache [num_blocks, ...]."""
    _need(block_ids, "block_ids", torch.int64)
    if not caches:
        return
    for c in caches:
        _need(c, "cache")
    per_block = caches[0][0].numel()
    ids = block_ids.contiguous()
    arr = _ptr_array(caches)
    _lib.check(_lib.load().swl_zero_blocks_bf16(arr, len(caches), _ptr(ids), ids.numel(), per_block, _stream()))


# ------------------------------------------------------- token-row ops ---
class RowSet:
    """A fixed list of per-token bf16 rows (1-D views of at least `width`
    elements each, 16-byte aligned), validated once and kept as a host array
    of device pointers so a decode loop can reuse it every step."""

    MAX_ROWS = 64

    def __init__(self, rows: Sequence[torch.Tensor], width: int):
        if len(rows) > self.MAX_ROWS:
            raise ValueError(f"at most {self.MAX_ROWS} rows")
        for i, r in enumerate(rows):
            _need(r, f"row[{i}]")
            if r.dim() != 1 or r.numel() < width or r.stride(0) != 1:
                raise ValueError(f"row[{i}] must be a contiguous 1-D view of >= {width} elements")
            if r.data_ptr() % 16:
                raise ValueError(f"row[{i}] must be 16-byte aligned")
        self.rows = list(rows)  # keeps the storage alive
        self.width = width
        self.array = _ptr_array(self.rows)

    def __len__(self):
        return len(self.rows)


def _rowset(rows, width: int) -> RowSet:
    if isinstance(rows, RowSet):
        if rows.width < width:
            raise ValueError(f"rows are {rows.width} wide, need {width}")
        return rows
    return RowSet(rows, width)


def rmsnorm_rows(h: torch.Tensor, weight: torch.Tensor, eps: float, out_rows, add_rows=None):
    """Residual stream h [ntok, d] (contiguous, updated in place): when
    add_rows is given h[t] = h[t] + add_rows[t] (bf16); then out_rows[t] =
    LlamaRMSNorm(h[t]) * weight."""
    _need(h, "h")
    _need(weight, "weight")
    if h.dim() != 2 or not h.is_contiguous():
        raise ValueError("h must be contiguous [ntok, d]")
    ntok, d = h.shape
    if weight.numel() != d or not weight.is_contiguous():
        raise ValueError("weight must be contiguous [d]")
    out = _rowset(out_rows, d)
    add = _rowset(add_rows, d) if add_rows is not None else None
    if len(out) != ntok or (add is not None and len(add) != ntok):
        raise ValueError("one out (and add) row per token")
    _lib.check(_lib.load().swl_rmsnorm_rows_bf16(_ptr(h), ntok, d, add.array if add is not None else None,
                                                 _ptr(weight), float(eps), out.array, _stream()))


def silu_mul_rows(in_rows, out_rows, inter: int):
    """out_rows[t] = silu(in_rows[t][:inter]) * in_rows[t][inter:2*inter]."""
    src = _rowset(in_rows, 2 * inter)
    dst = _rowset(out_rows, inter)
    if len(src) != len(dst):
        raise ValueError("one out row per in row")
    _lib.check(_lib.load().swl_silu_mul_rows_bf16(src.array, dst.array, len(src), inter, _stream()))


def _row_ptrs(t: torch.Tensor, c0: int, c1: int):
    """Host array of the device addresses of rows c0..c1 of a contiguous 2-D
    bf16 matrix (16-byte aligned rows when the base is and the width is a
    multiple of 8)."""
    base, step = t.data_ptr(), t.stride(0) * t.element_size()
    arr = (ctypes.c_void_p * (c1 - c0))()
    for i in range(c1 - c0):
        arr[i] = base + (c0 + i) * step
    return arr


def _rows_matrix(t: torch.Tensor, name: str) -> torch.Tensor:
    _need(t, name)
    m = t.reshape(-1, t.shape[-1])
    if not m.is_contiguous() or m.data_ptr() % 16 or m.shape[-1] % 8:
        raise ValueError(f"{name} must be contiguous, 16-byte aligned, last dim a multiple of 8")
    return m


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm of every row of x [..., d] into a new tensor (the
    worker's input / post-attention / final norms, worker_sync.py:1344-1350,
    :314-319), 64 rows per launch of the row kernel."""
    h = _rows_matrix(x, "x")
    _need(weight, "weight")
    n, d = h.shape
    if weight.numel() != d or not weight.is_contiguous():
        raise ValueError("weight must be contiguous [d]")
    out = torch.empty_like(x)
    o = out.view(n, d)
    lib, st = _lib.load(), _stream()
    for c0 in range(0, n, RowSet.MAX_ROWS):
        c1 = min(n, c0 + RowSet.MAX_ROWS)
        _lib.check(lib.swl_rmsnorm_rows_bf16(ctypes.c_void_p(h.data_ptr() + c0 * d * 2), c1 - c0, d, None,
                                             _ptr(weight), float(eps), _row_ptrs(o, c0, c1), st))
    return out


def silu_mul(gu: torch.Tensor, inter: int) -> torch.Tensor:
    """F.silu(gate) * up for a fused Gate+Up output gu [..., 2*inter] (gate
    columns first) into a new [..., inter] tensor (worker_sync.py:158)."""
    m = _rows_matrix(gu, "gu")
    n = m.shape[0]
    if m.shape[1] != 2 * inter:
        raise ValueError(f"gu must be [..., {2 * inter}]")
    out = torch.empty(*gu.shape[:-1], inter, dtype=gu.dtype, device=gu.device)
    o = out.view(n, inter)
    lib, st = _lib.load(), _stream()
    for c0 in range(0, n, RowSet.MAX_ROWS):
        c1 = min(n, c0 + RowSet.MAX_ROWS)
        _lib.check(lib.swl_silu_mul_rows_bf16(_row_ptrs(m, c0, c1), _row_ptrs(o, c0, c1), c1 - c0, inter, st))
    return out




def paged_attention_rows(qkv_rows, out_rows, q_len: int, hq: int, hkv: int, d: int, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, block_table: torch.Tensor, cache_seqlens: torch.Tensor,
                         positions: Optional[torch.Tensor], cos_sin: Optional[torch.Tensor], softmax_scale: float,
                         rope=True):
    """paged_attention over per-token rows: token t = seq * q_len + i has
    its fused [q | k | v] row at qkv_rows[t] (rotated in place) and gets its
    [hq * d] output at out_rows[t].  rope=2: q already rotated and k / v
    already appended by an out_mode 3 round (decode rows only)."""
    rope = 2 if rope == 2 else (1 if rope else 0)
    qkv = _rowset(qkv_rows, (hq + 2 * hkv) * d)
    out = _rowset(out_rows, hq * d)
    if len(qkv) != len(out) or len(qkv) % q_len:
        raise ValueError("rows must be nseq * q_len, one out row per qkv row")
    nseq = len(qkv) // q_len
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, nm)
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    _need(block_table, "block_table", torch.int32)
    _need(cache_seqlens, "cache_seqlens", torch.int32)
    nb, bs, hkv2, d2 = k_cache.shape
    if v_cache.shape != k_cache.shape or hkv2 != hkv or d2 != d:
        raise ValueError("cache geometry mismatch")
    if block_table.dim() != 2 or block_table.shape[0] < nseq or not block_table.is_contiguous():
        raise ValueError("block_table must be contiguous [nseq, max_blocks]")
    if cache_seqlens.numel() < nseq:
        raise ValueError("cache_seqlens must have nseq entries")
    max_pos = 0
    if rope == 1:
        _need(positions, "positions", torch.int64)
        _need(cos_sin, "cos_sin")
        if positions.numel() != nseq * q_len:
            raise ValueError("positions must have nseq * q_len entries")
        if cos_sin.shape[-1] != d or not cos_sin.is_contiguous():
            raise ValueError("cos_sin must be contiguous [max_pos, d]")
        max_pos = cos_sin.shape[0]
    rp = rope == 1
    _lib.check(_lib.load().swl_paged_attention_rows_bf16(
        qkv.array, out.array, nseq, q_len, hq, hkv, d, _ptr(k_cache), _ptr(v_cache), nb, bs, _ptr(block_table),
        block_table.shape[1], _ptr(cache_seqlens), _ptr(positions if rp else None),
        _ptr(cos_sin if rp else None), max_pos, rope, float(softmax_scale), _stream()))


# -------------------------------------------------------------- timing ---
def timer_arm(capacity: int):
    """Record HIP events around the next `capacity` decode-projection launches
    (base kernel and epilogue) issued outside graph capture."""
    _lib.check(_lib.load().swl_timer_arm(int(capacity)))


def timer_collect(max_records: int = 1 << 16):
    """Wait for the armed launches; returns a list of dicts with base_ms,
    epilogue_ms, n, k, ntok and the base kernel's algorithmic bytes."""
    m = int(max_records)
    fa, fb = (ctypes.c_float * m)(), (ctypes.c_float * m)()
    n, k, b = (ctypes.c_int64 * m)(), (ctypes.c_int64 * m)(), (ctypes.c_int64 * m)()
    t = (ctypes.c_int32 * m)()
    cnt = ctypes.c_int(0)
    _lib.check(_lib.load().swl_timer_collect(m, fa, fb, n, k, t, b, ctypes.byref(cnt)))
    return [{"base_ms": fa[i], "epilogue_ms": fb[i], "n": n[i], "k": k[i], "ntok": t[i], "bytes": b[i]}
            for i in range(cnt.value)]
