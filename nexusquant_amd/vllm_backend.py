"""vLLM page-granular caller and the decode-side consumer of compressed pages.

Mirrors nexusquant/integrations/vllm_backend.py (CompressedPage,
NexusQuantKVCompressor, NexusQuantPagedAttention) on the gfx950 library:

- compress_page        -> nq_page_encode  (vllm_backend.py:344-392)
- decompress_page      -> nq_page_decode  (:394-429)
- decompress_for_attention -> nq_page_logits (:431-467)
- pack/unpack_codes_nibble -> nq_nibble_pack / nq_nibble_unpack (:475-536)
- NexusQuantPagedAttention.forward -> nq_paged_attention (:692-765): decode
  attention read straight from the int8 pages, without materialising fp16
  keys or values.

Page format, arguments, return values and error messages are the reference's.
Every call needs the HIP library and device tensors; there is no CPU path.
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .hadamard import hadamard_constant
from .ops import _addr, _PtrArrays
from .rope import device_merged_table, device_table

_FP16_BYTES = 2
_KERNEL_HEAD_DIMS = (64, 128, 256)


@dataclasses.dataclass
class CompressedPage:
    """A single compressed KV block (vllm_backend.py:75-125).

    key_codes / value_codes: (num_heads, num_valid, head_dim) int8, 2 * lattice point
    key_scales / value_scales: (num_heads, num_valid) fp16 per-(head, token) scale
    positions: (num_valid,) int32 absolute token positions (RoPE of keys)
    num_valid: number of tokens stored
    max_position: largest stored position when known (set by compress_page;
    lets decoding size the RoPE table without reading the positions back).
    """

    key_codes: torch.Tensor
    value_codes: torch.Tensor
    key_scales: torch.Tensor
    value_scales: torch.Tensor
    positions: torch.Tensor
    num_valid: int
    max_position: Optional[int] = dataclasses.field(default=None, compare=False, repr=False)

    @property
    def compressed_bytes(self) -> int:
        n = self.num_valid
        h = self.key_codes.shape[0]
        d = self.key_codes.shape[2]
        return 2 * h * n * d + 2 * h * n * _FP16_BYTES + n * 4

    @property
    def uncompressed_bytes(self) -> int:
        n = self.num_valid
        h = self.key_codes.shape[0]
        d = self.key_codes.shape[2]
        return 2 * h * n * d * _FP16_BYTES


def _stream(dev) -> ctypes.c_void_p:
    return ctypes.c_void_p(_lib.current_stream_handle(dev))


def _page_max_position(page: CompressedPage) -> int:
    if page.max_position is None:
        pos = page.positions
        page.max_position = int(pos.max()) if pos.numel() else 0
        if pos.numel() and int(pos.min()) < 0:
            raise ValueError("page positions must be non-negative")
    return page.max_position


def _check_page(page: CompressedPage, head_dim: int) -> None:
    kc, vc = page.key_codes, page.value_codes
    for name, t, dt in (("key_codes", kc, torch.int8), ("value_codes", vc, torch.int8),
                        ("key_scales", page.key_scales, torch.float16),
                        ("value_scales", page.value_scales, torch.float16),
                        ("positions", page.positions, torch.int32)):
        _lib.require_device(t, f"CompressedPage.{name}")
        if t.dtype != dt:
            raise TypeError(f"CompressedPage.{name} must be {dt}, got {t.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"CompressedPage.{name} must be contiguous")
    if kc.dim() != 3 or kc.shape[2] != head_dim or vc.shape != kc.shape:
        raise ValueError(f"page codes must be (num_heads, tokens, {head_dim}), got {tuple(kc.shape)} / "
                         f"{tuple(vc.shape)}")
    h, n, _ = kc.shape
    if tuple(page.key_scales.shape) != (h, n) or tuple(page.value_scales.shape) != (h, n):
        raise ValueError("page scales must be (num_heads, tokens)")
    if tuple(page.positions.shape) != (n,):
        raise ValueError("page positions must be (tokens,)")
    if kc.data_ptr() % 8 or vc.data_ptr() % 8:
        raise ValueError("page codes must be 8-byte aligned")


class NexusQuantKVCompressor:
    """Compression backend for vLLM paged KV cache (vllm_backend.py:132-170).

    Keys: inverse RoPE at each token's absolute position -> Hadamard -> E8;
    values: Hadamard -> E8; int8 codes 2p and fp16 per-(head, token) scales.
    """

    def __init__(self, head_dim: int = 128, bits: int = 2, eviction_rate: float = 0.0,
                 rope_base: float = 10000.0):
        if bits not in (2, 3, 4):
            raise ValueError(f"bits must be 2, 3, or 4 (got {bits})")
        if head_dim & (head_dim - 1) != 0:
            raise ValueError(f"head_dim must be a power of 2 (got {head_dim})")
        if head_dim not in _KERNEL_HEAD_DIMS:
            raise NotImplementedError(f"head_dim {head_dim}: the gfx950 page kernels take 64, 128 or 256")
        self.head_dim = head_dim
        self.bits = bits
        self.levels = 2 ** bits
        self.eviction_rate = eviction_rate  # stored as the reference does; pages keep every token
        self.rope_base = rope_base

    # ------------------------------------------------------------------ tables

    def _tables(self, max_position: int, device):
        cos, sin = device_table(max_position + 1, self.head_dim, self.rope_base, None, device)
        dm, dp = device_merged_table(cos.shape[0], self.head_dim, self.rope_base, None, device)
        return cos, sin, dm, dp

    def _desc(self, n_pages: int, heads: int, tokens: int, is_key: bool, arrays: dict, tables,
              dtype_code: int = _lib.NQ_F16) -> _lib.PageDesc:
        cos = sin = dm = dp = None
        n_pos = 0
        if is_key:
            cos, sin, dm, dp = tables
            n_pos = cos.shape[0]
        return _lib.PageDesc(
            n_pages=n_pages, heads=heads, tokens=tokens, head_dim=self.head_dim, dtype=dtype_code,
            levels=self.levels, is_key=int(is_key), src=_addr(arrays.get("src")),
            positions=_addr(arrays.get("positions")), codes=_addr(arrays.get("codes")),
            scales=_addr(arrays.get("scales")), out=_addr(arrays.get("out")),
            rope_cos=_addr(cos), rope_sin=_addr(sin), rope_sin_minus_cos=_addr(dm), rope_cos_plus_sin=_addr(dp),
            rope_n_pos=n_pos, hadamard_scale=hadamard_constant(self.head_dim))

    # ------------------------------------------------------------- public API

    def compress_page(self, key_page: torch.Tensor, value_page: torch.Tensor,
                      page_positions: torch.Tensor) -> CompressedPage:
        """Compress one KV page (num_heads, block_size, head_dim) at absolute positions."""
        return self.compress_pages([(key_page, value_page, page_positions)])[0]

    def compress_pages(self, pages: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]
                       ) -> List[CompressedPage]:
        """compress_page over many pages; pages of equal shape share one launch per role."""
        lib = _lib.load()
        out: List[Optional[CompressedPage]] = [None] * len(pages)
        groups: Dict[tuple, List[int]] = {}
        prepared = []
        for i, (k, v, pos) in enumerate(pages):
            _lib.require_device(k, "key_page")
            if k.dim() != 3 or v.shape != k.shape:
                raise ValueError(f"key/value pages must be (num_heads, block_size, head_dim) of equal shape, "
                                 f"got {tuple(k.shape)} / {tuple(v.shape)}")
            h, n, d = k.shape
            if d != self.head_dim:
                raise ValueError(f"page head_dim {d} != compressor head_dim {self.head_dim}")
            dev = k.device
            pos_list = torch.as_tensor(pos)
            if pos_list.numel() != n:
                raise ValueError(f"page_positions has {pos_list.numel()} entries for {n} tokens")
            if n and pos_list.device.type == "cpu":
                lo, hi = int(pos_list.min()), int(pos_list.max())
            elif n:
                lo, hi = (int(x) for x in torch.stack([pos_list.min(), pos_list.max()]).tolist())
            else:
                lo = hi = 0
            if lo < 0:
                raise ValueError("page positions must be non-negative")
            pos_d = pos_list.to(device=dev, dtype=torch.int32).contiguous()
            _lib.require_device(v, "value_page")
            kk = k.contiguous()
            vv = v.contiguous()
            kk = kk if kk.data_ptr() % 16 == 0 else kk.clone()
            vv = vv if vv.data_ptr() % 16 == 0 else vv.clone()
            prepared.append((kk, vv, pos_d, hi))
            groups.setdefault((h, n, k.dtype, v.dtype, dev), []).append(i)
        for (h, n, kdt, vdt, dev), idx in groups.items():
            m = len(idx)
            kc = torch.empty(m, h, n, self.head_dim, dtype=torch.int8, device=dev).unbind(0)
            vc = torch.empty(m, h, n, self.head_dim, dtype=torch.int8, device=dev).unbind(0)
            ks = torch.empty(m, h, n, dtype=torch.float16, device=dev).unbind(0)
            vs = torch.empty(m, h, n, dtype=torch.float16, device=dev).unbind(0)
            max_pos = max(prepared[i][3] for i in idx)
            tables = self._tables(max_pos, dev)
            for role, is_key in (("k", True), ("v", False)):
                src = [prepared[i][0 if is_key else 1] for i in idx]
                codes = kc if is_key else vc
                scales = ks if is_key else vs
                groups_t = [src, [prepared[i][2] for i in idx] if is_key else None, list(codes), list(scales)]
                staged = _PtrArrays(groups_t, dev)
                arrays = dict(zip(("src", "positions", "codes", "scales"), staged.arrays))
                desc = self._desc(m, h, n, is_key, arrays, tables, _lib.dtype_code(kdt if is_key else vdt))
                with torch.cuda.device(dev):
                    try:
                        st = lib.nq_page_encode(ctypes.byref(desc), _stream(dev))
                    finally:
                        staged.release()
                _lib.check(st, "nq_page_encode")
            for j, i in enumerate(idx):
                out[i] = CompressedPage(key_codes=kc[j], value_codes=vc[j], key_scales=ks[j], value_scales=vs[j],
                                        positions=prepared[i][2], num_valid=n, max_position=prepared[i][3])
        return out  # type: ignore[return-value]

    def decompress_page(self, compressed_page: CompressedPage) -> Tuple[torch.Tensor, torch.Tensor]:
        """(keys, values) (num_heads, tokens, head_dim) fp16 of one page."""
        return self.decompress_pages([compressed_page])[0]

    def decompress_pages(self, pages: Sequence[CompressedPage]) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        lib = _lib.load()
        out: List[Optional[Tuple[torch.Tensor, torch.Tensor]]] = [None] * len(pages)
        groups: Dict[tuple, List[int]] = {}
        for i, p in enumerate(pages):
            _check_page(p, self.head_dim)
            h, n, _ = p.key_codes.shape
            groups.setdefault((h, n, p.key_codes.device), []).append(i)
        for (h, n, dev), idx in groups.items():
            m = len(idx)
            ko = torch.empty(m, h, n, self.head_dim, dtype=torch.float16, device=dev).unbind(0)
            vo = torch.empty(m, h, n, self.head_dim, dtype=torch.float16, device=dev).unbind(0)
            if n:
                tables = self._tables(max(_page_max_position(pages[i]) for i in idx), dev)
                for is_key in (True, False):
                    pg = [pages[i] for i in idx]
                    groups_t = [[p.key_codes if is_key else p.value_codes for p in pg],
                                [p.key_scales if is_key else p.value_scales for p in pg],
                                [p.positions for p in pg] if is_key else None,
                                list(ko if is_key else vo)]
                    staged = _PtrArrays(groups_t, dev)
                    arrays = dict(zip(("codes", "scales", "positions", "out"), staged.arrays))
                    desc = self._desc(m, h, n, is_key, arrays, tables)
                    with torch.cuda.device(dev):
                        try:
                            st = lib.nq_page_decode(ctypes.byref(desc), _stream(dev))
                        finally:
                            staged.release()
                    _lib.check(st, "nq_page_decode")
            for j, i in enumerate(idx):
                out[i] = (ko[j], vo[j])
        return out  # type: ignore[return-value]

    def decompress_for_attention(self, compressed_page: CompressedPage, query: torch.Tensor) -> torch.Tensor:
        """Logits (num_heads, q_len, tokens) fp32 = q . k / sqrt(head_dim) against the page's keys."""
        lib = _lib.load()
        p = compressed_page
        _check_page(p, self.head_dim)
        _lib.require_device(query, "query")
        h, n, d = p.key_codes.shape
        if query.dim() != 3 or query.shape[0] != h or query.shape[2] != d:
            raise ValueError(f"query must be (num_heads={h}, q_len, head_dim={d}), got {tuple(query.shape)}")
        dev = p.key_codes.device
        q = query.contiguous()
        if q.data_ptr() % 16:
            q = q.clone()
        q_len = q.shape[1]
        logits = torch.empty(h, q_len, n, dtype=torch.float32, device=dev)
        if n == 0 or q_len == 0:
            return logits
        tables = self._tables(_page_max_position(p), dev)
        staged = _PtrArrays([[p.key_codes], [p.key_scales], [p.positions]], dev)
        arrays = dict(zip(("codes", "scales", "positions"), staged.arrays))
        desc = self._desc(1, h, n, True, arrays, tables)
        with torch.cuda.device(dev):
            try:
                st = lib.nq_page_logits(ctypes.byref(desc), _addr(q), _lib.dtype_code(q.dtype), q_len,
                                        ctypes.c_float(float(np.float32(math.sqrt(self.head_dim)))),
                                        _addr(logits), _stream(dev))
            finally:
                staged.release()
        _lib.check(st, "nq_page_logits")
        return logits

    @staticmethod
    def pack_codes_nibble(codes: torch.Tensor) -> torch.Tensor:
        """(..., d) int8 -> (..., ceil(d/2)) uint8: clamp(code + 8, 0, 15) nibbles, low nibble first."""
        lib = _lib.load()
        _lib.require_device(codes, "codes")
        if codes.dtype != torch.int8:
            raise TypeError(f"codes must be int8, got {codes.dtype}")
        d = codes.shape[-1]
        c = codes.contiguous()
        rows = c.numel() // d if d else 0
        out = torch.empty(*codes.shape[:-1], (d + 1) // 2, dtype=torch.uint8, device=codes.device)
        if rows and d:
            with torch.cuda.device(codes.device):
                st = lib.nq_nibble_pack(_addr(c), rows, d, _addr(out), _stream(codes.device))
            _lib.check(st, "nq_nibble_pack")
        return out

    @staticmethod
    def unpack_codes_nibble(packed: torch.Tensor, original_d: int) -> torch.Tensor:
        """Inverse of pack_codes_nibble: (..., ceil(d/2)) uint8 -> (..., original_d) int8."""
        lib = _lib.load()
        _lib.require_device(packed, "packed")
        if packed.dtype != torch.uint8:
            raise TypeError(f"packed codes must be uint8, got {packed.dtype}")
        pc = packed.shape[-1]
        d = min(int(original_d), 2 * pc)
        p = packed.contiguous()
        rows = p.numel() // pc if pc else 0
        out = torch.empty(*packed.shape[:-1], max(d, 0), dtype=torch.int8, device=packed.device)
        if rows and d > 0:
            with torch.cuda.device(packed.device):
                st = lib.nq_nibble_unpack(_addr(p), rows, pc, d, _addr(out), _stream(packed.device))
            _lib.check(st, "nq_nibble_unpack")
        return out

    def compression_ratio(self, page: CompressedPage) -> float:
        if page.uncompressed_bytes == 0:
            return 1.0
        return page.uncompressed_bytes / page.compressed_bytes


# ---------------------------------------------------------------------------
# Decode attention over compressed pages
# ---------------------------------------------------------------------------

def build_chunk_plan(rows: Sequence[Sequence[Tuple[int, int]]], context_lens: Sequence[int], chunk_cap: int):
    """Cut each row's token stream into chunks of at most chunk_cap tokens.

    rows[b] lists (slot, tokens) of the pages row b reads, in order; row b
    attends to the first context_lens[b] tokens of their concatenation (Python
    slice semantics: a negative length drops tokens from the end, 0 none).
    Returns the int32 arrays of nq_attn_desc (segs, units, chunk_units,
    chunk_row, chunk_tokens, row_chunks) and the total token count.
    """
    segs: List[Tuple[int, int, int, int]] = []
    units: List[Tuple[int, int]] = []
    chunk_units: List[int] = []
    chunk_row: List[int] = []
    chunk_tokens: List[int] = []
    row_chunks = [0]
    total = 0
    for b, row in enumerate(rows):
        ctx = int(context_lens[b])
        avail = sum(n for _, n in row)
        use = 0 if ctx == 0 else (ctx if ctx > 0 else avail + ctx)
        use = max(0, min(use, avail))
        fill = None  # tokens in the row's open chunk (None: none open)
        for slot, n_page in row:
            if use == 0:
                break
            n = min(n_page, use)
            use -= n
            t = 0
            while t < n:
                if fill is None or fill == chunk_cap:
                    chunk_units.append(len(units))
                    chunk_row.append(b)
                    chunk_tokens.append(0)
                    fill = 0
                take = min(n - t, chunk_cap - fill)
                seg = len(segs)
                segs.append((slot, t, take, fill))
                units.extend((seg, u) for u in range(0, take, 16))
                fill += take
                chunk_tokens[-1] += take
                total += take
                t += take
        row_chunks.append(len(chunk_row))
    chunk_units.append(len(units))
    parts = {
        "segs": np.array(segs, dtype=np.int32).reshape(-1),
        "units": np.array(units, dtype=np.int32).reshape(-1),
        "chunk_units": np.array(chunk_units, dtype=np.int32),
        "chunk_row": np.array(chunk_row, dtype=np.int32),
        "chunk_tokens": np.array(chunk_tokens, dtype=np.int32),
        "row_chunks": np.array(row_chunks, dtype=np.int32),
    }
    return parts, total


def unit_records(parts: dict, slot_pages: Sequence[CompressedPage], head_dim: int) -> np.ndarray:
    """The 16-int32 unit records of nq_attn_desc from a chunk plan's segments
    and units: absolute addresses of each unit's first token in its page."""
    segs = parts["segs"].reshape(-1, 4).astype(np.int64)
    units = parts["units"].reshape(-1, 2).astype(np.int64)
    rec = np.zeros((len(units), 16), dtype=np.int64)
    if len(units):
        base = np.array([[p.key_codes.data_ptr(), p.value_codes.data_ptr(), p.key_scales.data_ptr(),
                          p.value_scales.data_ptr(), p.positions.data_ptr(), p.key_codes.shape[1]]
                         for p in slot_pages], dtype=np.int64).reshape(-1, 6)
        sg = segs[units[:, 0]]
        slot, first, n, off = sg[:, 0], sg[:, 1], sg[:, 2], sg[:, 3]
        t0 = first + units[:, 1]
        b = base[slot]
        addr = np.stack([b[:, 0] + t0 * head_dim, b[:, 1] + t0 * head_dim, b[:, 2] + 2 * t0,
                         b[:, 3] + 2 * t0, b[:, 4] + 4 * t0], axis=1)
        rec[:, 0:10:2] = addr & 0xFFFFFFFF
        rec[:, 1:10:2] = addr >> 32
        rec[:, 10] = b[:, 5]
        rec[:, 11] = np.minimum(16, n - units[:, 1])
        rec[:, 12] = off + units[:, 1]
    return rec.astype(np.uint32).view(np.int32).reshape(-1)


@dataclasses.dataclass
class PagedAttentionPlan:
    """Device description of which page tokens each batch row attends to
    (the chunk plan of nq_paged_attention), reusable across decode steps while
    the pages, block tables and context lengths stay the same."""
    batch: int
    kv_heads: int
    head_dim: int
    n_chunks: int
    ints: Optional[torch.Tensor]       # int32: unit records and index arrays, see offsets
    offsets: Dict[str, int]
    max_position: int
    keepalive: list                    # the pages whose memory the plan points at
    tokens: int                        # tokens attended over all rows


class NexusQuantPagedAttention:
    """Paged attention over compressed pages (vllm_backend.py:543-775)."""

    def __init__(self, compressor: NexusQuantKVCompressor):
        self.compressor = compressor
        self._block_pool: dict = {}
        self._next_block_id: int = 0

    def allocate_block(self) -> int:
        block_id = self._next_block_id
        self._next_block_id += 1
        return block_id

    def free_block(self, block_id: int) -> None:
        self._block_pool.pop(block_id, None)

    def is_block_compressed(self, block_id: int) -> bool:
        return block_id in self._block_pool

    def compress_and_cache(self, key: torch.Tensor, value: torch.Tensor, key_cache: dict, value_cache: dict,
                           slot_mapping: torch.Tensor) -> None:
        """reshape_and_cache for compressed storage (vllm_backend.py:622-688): the new tokens of each
        block become that block's page, at positions = their slot offsets."""
        if key.shape[0] == 0:
            return
        block_size = self._infer_block_size(slot_mapping)
        device = key.device
        block_ids = (slot_mapping // block_size).tolist()
        offsets = (slot_mapping % block_size).tolist()
        tok_idx: Dict[int, list] = {}
        tok_off: Dict[int, list] = {}
        for i, (bid, off) in enumerate(zip(block_ids, offsets)):
            tok_idx.setdefault(bid, []).append(i)
            tok_off.setdefault(bid, []).append(off)
        work = []
        for bid, idx in tok_idx.items():
            t = torch.tensor(idx, dtype=torch.long, device=device)
            work.append((key[t].permute(1, 0, 2), value[t].permute(1, 0, 2),
                         torch.tensor(tok_off[bid], dtype=torch.int32)))
        pages = self.compressor.compress_pages(work)
        for bid, page in zip(tok_idx.keys(), pages):
            key_cache[bid] = page
            value_cache[bid] = page

    # --------------------------------------------------------------- forward

    def plan(self, compressed_key_cache: dict, block_tables: List[List[int]], context_lens) -> PagedAttentionPlan:
        """Chunk plan of the tokens each row attends to: the pages of block_tables[b]
        present in the cache, concatenated, first context_lens[b] tokens (Python
        slice semantics, as the reference slices the concatenation)."""
        chunk_cap = int(_lib.load().nq_paged_attention_chunk_tokens())
        ctx = [int(x) for x in (context_lens.tolist() if torch.is_tensor(context_lens) else context_lens)]
        slot_of: Dict[int, int] = {}
        slot_pages: List[CompressedPage] = []
        rows = []
        kv_heads = head_dim = None
        for b in range(len(ctx)):
            row = []
            if ctx[b] != 0:
                for bid in block_tables[b]:
                    p = compressed_key_cache.get(bid) if bid in compressed_key_cache else None
                    if p is None:
                        continue
                    if kv_heads is None:
                        kv_heads, head_dim = p.key_codes.shape[0], p.key_codes.shape[2]
                        if head_dim != self.compressor.head_dim:
                            raise ValueError(f"page head_dim {head_dim} != compressor head_dim "
                                             f"{self.compressor.head_dim}")
                    if p.key_codes.shape[0] != kv_heads or p.key_codes.shape[2] != head_dim:
                        raise ValueError("all pages must share (num_heads, head_dim)")
                    if id(p) not in slot_of:
                        _check_page(p, head_dim)
                        slot_of[id(p)] = len(slot_pages)
                        slot_pages.append(p)
                    row.append((slot_of[id(p)], p.key_codes.shape[1]))
            rows.append(row)
        parts, total = build_chunk_plan(rows, ctx, chunk_cap)
        n_chunks = len(parts["chunk_row"])
        dev = None
        max_pos = 0
        if slot_pages:
            dev = slot_pages[0].key_codes.device
            for p in slot_pages:
                max_pos = max(max_pos, _page_max_position(p))
        parts["units"] = unit_records(parts, slot_pages, head_dim or self.compressor.head_dim)
        offsets: Dict[str, int] = {}
        buf = []
        at = 0
        for k in ("units", "chunk_units", "chunk_row", "chunk_tokens", "row_chunks"):
            v = parts[k]
            offsets[k] = at
            pad = (-len(v)) % 4  # 16-byte aligned starts
            buf.append(v)
            if pad:
                buf.append(np.zeros(pad, dtype=np.int32))
            at += len(v) + pad
        if dev is None and torch.cuda.is_available():
            dev = torch.device("cuda", torch.cuda.current_device())
        ints = torch.tensor(np.concatenate(buf), device=dev) if dev is not None else None
        return PagedAttentionPlan(batch=len(ctx), kv_heads=kv_heads or 0,
                                  head_dim=head_dim or self.compressor.head_dim, n_chunks=n_chunks,
                                  ints=ints, offsets=offsets, max_position=max_pos,
                                  keepalive=slot_pages, tokens=total)

    def run(self, plan: PagedAttentionPlan, query: torch.Tensor, out: Optional[torch.Tensor] = None,
            workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Attention of query (batch, num_heads, head_dim) over a plan's tokens."""
        lib = _lib.load()
        _lib.require_device(query, "query")
        if query.dim() != 3 or query.shape[0] != plan.batch:
            raise ValueError(f"query must be (batch={plan.batch}, num_heads, head_dim), got {tuple(query.shape)}")
        b, hq, d = query.shape
        if d != self.compressor.head_dim:
            raise ValueError(f"query head_dim {d} != compressor head_dim {self.compressor.head_dim}")
        dev = query.device
        q = query.contiguous()
        if q.data_ptr() % 16:
            q = q.clone()
        if out is None:
            out = torch.empty_like(q)
        kv = plan.kv_heads if plan.n_chunks else hq
        if hq % kv:
            raise ValueError(f"num_heads {hq} is not a multiple of the pages' num_heads {kv}")
        ws_bytes = lib.nq_paged_attention_workspace(plan.n_chunks, hq, d)
        if workspace is None or workspace.numel() < ws_bytes:
            from .ops import workspace as stream_workspace
            workspace = stream_workspace(dev, ws_bytes)
        cos = sin = dm = dp = None
        n_pos = 0
        if plan.n_chunks:
            cos, sin, dm, dp = self.compressor._tables(plan.max_position, dev)
            n_pos = cos.shape[0]
        ints = plan.ints
        base = ints.data_ptr() if ints is not None else 0

        def at(name):
            return ctypes.c_void_p(base + 4 * plan.offsets[name]) if ints is not None else None

        desc = _lib.AttnDesc(
            batch=b, q_heads=hq, kv_heads=kv, head_dim=d, q_dtype=_lib.dtype_code(q.dtype),
            n_chunks=plan.n_chunks, query=_addr(q), out=_addr(out), units=at("units"),
            chunk_units=at("chunk_units"),
            chunk_row=at("chunk_row"), chunk_tokens=at("chunk_tokens"), row_chunks=at("row_chunks"),
            rope_cos=_addr(cos), rope_sin=_addr(sin), rope_sin_minus_cos=_addr(dm), rope_cos_plus_sin=_addr(dp),
            rope_n_pos=n_pos, hadamard_scale=hadamard_constant(d),
            scale_divisor=float(np.float32(math.sqrt(d))), workspace=_addr(workspace), workspace_bytes=ws_bytes)
        with torch.cuda.device(dev):
            st = lib.nq_paged_attention(ctypes.byref(desc), _stream(dev))
        _lib.check(st, "nq_paged_attention")
        return out

    def forward(self, query: torch.Tensor, compressed_key_cache: dict, compressed_value_cache: dict,
                block_tables: List[List[int]], context_lens: torch.Tensor) -> torch.Tensor:
        """(batch, num_heads, head_dim) attended output, the query's dtype (fp16-rounded values)."""
        plan = self.plan(compressed_key_cache, block_tables, context_lens)
        return self.run(plan, query)

    @staticmethod
    def _infer_block_size(slot_mapping: torch.Tensor) -> int:
        """The reference's heuristic (vllm_backend.py:775-786), kept as is: the first
        candidate always passes, so it returns 4 for any non-empty mapping."""
        if slot_mapping.numel() == 0:
            return 16
        for bs in [4, 8, 16, 32]:
            if (slot_mapping % bs).max() < bs:
                return bs
        return 16
