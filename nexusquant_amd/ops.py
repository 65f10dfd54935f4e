"""Tensor-level wrappers of the gfx950 kernels (device tensors in, device tensors out)."""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib
from .hadamard import hadamard_constant, next_power_of_2
from .rope import device_merged_table, device_table

SYM_BITS = {2: 2, 4: 3, 8: 4, 16: 5}


@dataclass
class PackedCodes:
    """Lossless packed relaxed-E8 codes of one [batch, heads, seq, head_dim] tensor.

    syms   uint8 [batch, heads, seq, D/8 * bits]  (bits = 2,3,4,5 for levels 2,4,8,16)
    cosets uint8 [batch, heads, seq, D/64]        (bit g: group g is a half-integer point)
    scales fp32  [batch, heads, seq]
    D is head_dim padded to a power of two.  Slot k of a row's symbol bytes holds
    group 4*(k mod D/32) + (k div D/32); symbol j of a group sits at bit j*bits.
    """
    syms: torch.Tensor
    cosets: torch.Tensor
    scales: torch.Tensor
    levels: int
    head_dim: int
    padded_dim: int
    is_key: bool

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.syms, self.cosets, self.scales))


class _AddressRing:
    """Per-device ring of pinned host and device int64 slots for the address
    arrays a launch descriptor points at.

    Each launch writes its addresses into a free span of the pinned buffer and
    copies the span to the same span of the device buffer with one asynchronous
    copy on the launch stream.  An event recorded after the launch marks the
    span busy; a span is rewritten only after its event has completed, which
    the host checks (and in practice never waits for: the ring holds 64K
    addresses).  Allocating pinned memory per launch instead would let the
    runtime synchronise the device, and a pageable copy would block the host
    behind the previous kernel.
    """

    ENTRIES = 1 << 16
    EVENTS = 16  # events created (and recorded once) up front

    def __init__(self, device):
        self.device = device
        self.host = torch.empty(self.ENTRIES, dtype=torch.int64, pin_memory=True)
        self.host_np = self.host.numpy()
        self.dev = torch.empty(self.ENTRIES, dtype=torch.int64, device=device)
        self.head = 0
        self.busy: List[Tuple[int, int, torch.cuda.Event]] = []  # oldest first
        # The runtime creates an event's resources at its first record, which can
        # block the host; recording a pool once here keeps that out of launches.
        stream = torch.cuda.current_stream(device)
        self.free_events: List[torch.cuda.Event] = []
        for _ in range(self.EVENTS):
            ev = torch.cuda.Event()
            ev.record(stream)
            self.free_events.append(ev)
        self.lock = threading.Lock()

    def _wait_for(self, start: int, end: int) -> None:
        # recycle completed reservations, oldest first
        while self.busy and self.busy[0][2].query():
            self.free_events.append(self.busy.pop(0)[2])
        keep = []
        for (s0, e0, ev) in self.busy:
            if s0 < end and start < e0:
                ev.synchronize()
                self.free_events.append(ev)
            else:
                keep.append((s0, e0, ev))
        self.busy = keep

    def stage(self, flat: List[int]) -> Tuple[torch.Tensor, Tuple[int, int]]:
        n = len(flat)
        if n > self.ENTRIES:
            raise ValueError(f"{n} tensors in one launch exceed the address ring ({self.ENTRIES})")
        with self.lock:
            start = self.head if self.head + n <= self.ENTRIES else 0
            end = start + n
            self._wait_for(start, end)
            self.host_np[start:end] = flat
            self.dev[start:end].copy_(self.host[start:end], non_blocking=True)
            self.head = end
        return self.dev[start:end], (start, end)

    def release(self, span: Tuple[int, int]) -> None:
        with self.lock:
            ev = self.free_events.pop() if self.free_events else torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
            self.busy.append((span[0], span[1], ev))


_rings: Dict[int, _AddressRing] = {}
_rings_lock = threading.Lock()


def _ring(device) -> _AddressRing:
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    r = _rings.get(idx)
    if r is None:
        with _rings_lock:
            r = _rings.get(idx)
            if r is None:
                r = _rings[idx] = _AddressRing(torch.device("cuda", idx))
    return r


class _PtrArrays:
    """Device int64 arrays of the base addresses of each tensor group, staged
    through the device's address ring.  Call release() right after the launch
    that reads them."""

    def __init__(self, groups: Sequence[Optional[Sequence[torch.Tensor]]], device):
        flat: List[int] = []
        spans = []
        for g in groups:
            if g is None:
                spans.append(None)
                continue
            spans.append((len(flat), len(g)))
            flat.extend(t.data_ptr() for t in g)
        self._ring = None
        self._span = None
        if not flat:
            self.arrays = [None for _ in groups]
            return
        self._ring = _ring(device)
        dev, self._span = self._ring.stage(flat)
        self.arrays = [None if sp is None else dev[sp[0]:sp[0] + sp[1]] for sp in spans]

    def release(self) -> None:
        if self._ring is not None and self._span is not None:
            self._ring.release(self._span)
            self._span = None


def _addr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_workspaces: Dict[Tuple[int, int], torch.Tensor] = {}
_workspaces_lock = threading.Lock()


def workspace(device, nbytes: int) -> torch.Tensor:
    """A device byte buffer of at least nbytes for the current stream of `device`,
    kept between calls (grown when a call needs more).  Calls on one stream run
    in stream order, so they can share it; each stream has its own.  Freed by
    release_workspaces()."""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, _lib.current_stream_handle(torch.device("cuda", idx)))
    n = max(int(nbytes), 1)
    with _workspaces_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() < n:
            # round up to 1 MiB so that slowly growing shapes do not reallocate each call
            buf = torch.empty(((n + (1 << 20) - 1) >> 20) << 20, dtype=torch.uint8, device=torch.device("cuda", idx))
            _workspaces[key] = buf
    return buf


def release_workspaces() -> None:
    """Drop the cached workspaces (their memory returns to torch's allocator)."""
    with _workspaces_lock:
        _workspaces.clear()


def quantize_tensors(tensors: Sequence[torch.Tensor], *, is_key: bool, levels: int,
                     rope_base: float = 10000.0, rope_scaling: Optional[dict] = None,
                     gather: Optional[torch.Tensor] = None, keep: Optional[torch.Tensor] = None,
                     keep_mode: int = _lib.NQ_KEEP_ZERO, recon_out: Optional[Sequence[torch.Tensor]] = None,
                     recon: bool = True, codes: bool = False, launch_events=None, merged_tables: bool = True,
                     order: Optional[torch.Tensor] = None, n_kept: Optional[torch.Tensor] = None,
                     ) -> Tuple[Optional[List[torch.Tensor]], Optional[List[PackedCodes]]]:
    """Run the fused quantizer over same-shaped [b, h, s, d] tensors in one launch.

    gather: int32/int64 [b, seq_out] source token per output row (truncation).
    keep:   bool/uint8 [b, seq_in]; with keep_mode NQ_KEEP_ZERO rows with keep == 0
            are zeroed (mask eviction); NQ_KEEP_WRITE_KEPT / NQ_KEEP_WRITE_EVICTED
            write only the kept / only the evicted rows (soft eviction).
    recon_out: fp16 [b, h, seq_out, d] tensors to write the reconstructions into
            (rows this launch does not write keep their contents).
    launch_events: optional (start, end) torch.cuda.Event pair recorded on the
    launch stream immediately around the kernel launch.
    merged_tables: pass the precomputed fl(sin - cos) / fl(cos + sin) tables for
            keys (False: the kernel forms them from cos / sin; same results).
    order, n_kept: keep_mask()'s kept_idx [b, seq] (kept positions first, then
            the evicted ones) and n_kept [b], with `keep` and keep_mode
            NQ_KEEP_ZERO: only the kept rows are read and quantized; evicted rows
            get the zero-row outputs directly.  Same results as without them.
    Returns (fp16 reconstructions or None, PackedCodes or None), one per tensor.
    """
    lib = _lib.load()
    if not tensors:
        return ([] if recon else None), ([] if codes else None)
    t0 = tensors[0]
    _lib.require_device(t0, "KV tensor")
    if t0.dim() != 4:
        raise ValueError(f"expected [batch, heads, seq, head_dim] tensors, got shape {tuple(t0.shape)}")
    b, h, s, d = t0.shape
    for t in tensors:
        if t.shape != t0.shape or t.dtype != t0.dtype or t.device != t0.device:
            raise ValueError("all tensors of one launch must share shape, dtype and device")
    if levels not in SYM_BITS:
        raise ValueError(f"levels must be 2, 4, 8 or 16, got {levels}")
    D = next_power_of_2(d)
    if d not in (64, 96, 128, 256):
        raise NotImplementedError(f"head_dim {d} is not supported by the fused kernel (64, 96, 128, 256)")
    dev = t0.device
    # contiguous and 16-byte aligned (the kernel reads 16-byte vectors)
    src = [t.contiguous() for t in tensors]
    src = [t if t.data_ptr() % 16 == 0 else t.clone() for t in src]
    seq_out = s
    g = None
    if gather is not None:
        g = gather.to(device=dev, dtype=torch.int32).contiguous()
        if g.dim() == 1:
            g = g.unsqueeze(0).expand(b, -1).contiguous()
        if g.shape[0] != b:
            raise ValueError(f"gather must be [batch, seq_out], got {tuple(g.shape)}")
        seq_out = g.shape[1]
        if g.numel() and (int(g.min()) < 0 or int(g.max()) >= s):
            raise ValueError(f"gather indices must lie in [0, {s})")
    k = None
    if keep is not None:
        k = keep.to(device=dev, dtype=torch.uint8).contiguous()
        if tuple(k.shape) != (b, s):
            raise ValueError(f"keep must be [batch, seq] = {(b, s)}, got {tuple(k.shape)}")

    if keep_mode not in (_lib.NQ_KEEP_ZERO, _lib.NQ_KEEP_WRITE_KEPT, _lib.NQ_KEEP_WRITE_EVICTED):
        raise ValueError(f"unknown keep_mode {keep_mode}")
    if keep_mode != _lib.NQ_KEEP_ZERO and k is None:
        raise ValueError("keep_mode other than NQ_KEEP_ZERO needs a keep mask")
    o = nk = None
    if order is not None:
        if k is None or keep_mode != _lib.NQ_KEEP_ZERO or g is not None or n_kept is None:
            raise ValueError("a row list (order) takes a keep mask, n_kept, keep_mode NQ_KEEP_ZERO and no gather")
        o = order.to(device=dev, dtype=torch.int32).contiguous()
        nk = n_kept.to(device=dev, dtype=torch.int32).contiguous()
        if tuple(o.shape) != (b, s) or tuple(nk.shape) != (b,):
            raise ValueError(f"order must be [batch, seq] = {(b, s)} and n_kept [batch], got "
                             f"{tuple(o.shape)} and {tuple(nk.shape)}")
    n = len(src)
    # one allocation per output kind; every tensor gets a contiguous slice
    recon_t = None
    if recon_out is not None:
        recon_t = list(recon_out)
        if len(recon_t) != n:
            raise ValueError("recon_out must hold one tensor per input tensor")
        for r in recon_t:
            _lib.require_device(r, "recon_out tensor")
            if (tuple(r.shape) != (b, h, seq_out, d) or r.dtype != torch.float16 or not r.is_contiguous()
                    or r.data_ptr() % 16):
                raise ValueError(f"recon_out tensors must be contiguous 16-byte aligned fp16 {(b, h, seq_out, d)}")
    elif recon:
        recon_t = list(torch.empty(n, b, h, seq_out, d, dtype=torch.float16, device=dev).unbind(0))
    codes_t = None
    if codes:
        syms = torch.empty(n, b, h, seq_out, D // 8 * SYM_BITS[levels], dtype=torch.uint8, device=dev).unbind(0)
        cosets = torch.empty(n, b, h, seq_out, D // 64, dtype=torch.uint8, device=dev).unbind(0)
        scales = torch.empty(n, b, h, seq_out, dtype=torch.float32, device=dev).unbind(0)
        codes_t = [PackedCodes(syms=syms[i], cosets=cosets[i], scales=scales[i], levels=levels, head_dim=d,
                               padded_dim=D, is_key=is_key) for i in range(n)]

    cos = sin = dm = dp = None
    n_pos = 0
    if is_key:
        cos, sin = device_table(max(s, seq_out), d, rope_base, rope_scaling, dev)
        n_pos = cos.shape[0]
        if d != 96 and merged_tables:  # power-of-two head dims fold RoPE into the top Hadamard stage
            dm, dp = device_merged_table(n_pos, d, rope_base, rope_scaling, dev)

    names = ("src", "recon", "syms", "cosets", "scales")
    groups = [src, recon_t,
              [c.syms for c in codes_t] if codes_t else None,
              [c.cosets for c in codes_t] if codes_t else None,
              [c.scales for c in codes_t] if codes_t else None]
    staged = _PtrArrays(groups, dev)
    arrays = dict(zip(names, staged.arrays))
    desc = _lib.QuantDesc(
        n_tensors=n, batch=b, heads=h, seq_in=s, seq_out=seq_out, head_dim=d,
        dtype=_lib.dtype_code(t0.dtype), levels=levels, is_key=int(is_key), keep_mode=keep_mode,
        src=_addr(arrays["src"]), recon=_addr(arrays["recon"]), syms=_addr(arrays["syms"]),
        cosets=_addr(arrays["cosets"]), scales=_addr(arrays["scales"]),
        gather=_addr(g), keep=_addr(k), rope_cos=_addr(cos), rope_sin=_addr(sin),
        rope_n_pos=n_pos, hadamard_scale=hadamard_constant(D),
        rope_sin_minus_cos=_addr(dm), rope_cos_plus_sin=_addr(dp), order=_addr(o), n_kept=_addr(nk))
    with torch.cuda.device(dev):
        try:
            if launch_events is not None:
                launch_events[0].record()
            status = lib.nq_quantize(ctypes.byref(desc), ctypes.c_void_p(_lib.current_stream_handle(dev)))
            if launch_events is not None:
                launch_events[1].record()
        finally:
            staged.release()
    _lib.check(status, "nq_quantize")
    return recon_t, codes_t


# ---------------------------------------------------------------------------
# Eviction: importance, keep mask, fp16 passthrough
# ---------------------------------------------------------------------------

def score_keykey(keys: torch.Tensor, obs_window: int = 32) -> torch.Tensor:
    """Key-key importance [batch, seq] fp32 of keys [batch, heads, seq, d] (MFMA kernel)."""
    lib = _lib.load()
    _lib.require_device(keys, "keys")
    if keys.dim() != 4:
        raise ValueError(f"expected keys [batch, heads, seq, head_dim], got {tuple(keys.shape)}")
    b, h, s, d = keys.shape
    k = keys.contiguous()
    if k.data_ptr() % 16:
        k = k.clone()
    dev = k.device
    imp = torch.empty(b, s, dtype=torch.float32, device=dev)
    if s == 0:
        return imp
    if int(obs_window) <= 0:
        raise ValueError(f"obs_window must be positive, got {obs_window}")
    ws_bytes = lib.nq_score_keykey_workspace(b, h, s, int(obs_window))
    ws = workspace(dev, ws_bytes)
    scale = float(d) ** -0.5
    with torch.cuda.device(dev):
        st = lib.nq_score_keykey(_addr(k), _lib.dtype_code(k.dtype), b, h, s, d, int(obs_window),
                                 ctypes.c_float(scale), _addr(imp), _addr(ws), ws_bytes,
                                 ctypes.c_void_p(_lib.current_stream_handle(dev)))
    _lib.check(st, "nq_score_keykey")
    return imp


def score_keykey_noalloc(keys: torch.Tensor, obs_window: int = 32,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """score_keykey through nq_score_keykey_noalloc: the library's static
    per-GPU scratch instead of a workspace, so the launch allocates nothing
    (pass `out`, fp32 [batch, seq], to allocate nothing here either).  keys
    must be contiguous and 16-byte aligned.  Calls that overlap on one GPU
    share the scratch and race."""
    lib = _lib.load()
    _lib.require_device(keys, "keys")
    if keys.dim() != 4 or not keys.is_contiguous() or keys.data_ptr() % 16:
        raise ValueError("keys must be a contiguous, 16-byte aligned [batch, heads, seq, head_dim] tensor")
    b, h, s, d = keys.shape
    if out is None:
        out = torch.empty(b, s, dtype=torch.float32, device=keys.device)
    elif (tuple(out.shape) != (b, s) or out.dtype != torch.float32 or not out.is_contiguous()
          or out.device != keys.device):
        raise ValueError(f"out must be a contiguous fp32 [{b}, {s}] tensor on {keys.device}")
    if s == 0:
        return out
    with torch.cuda.device(keys.device):
        st = lib.nq_score_keykey_noalloc(_addr(keys), _lib.dtype_code(keys.dtype), b, h, s, d, int(obs_window),
                                         ctypes.c_float(float(d) ** -0.5), _addr(out),
                                         ctypes.c_void_p(_lib.current_stream_handle(keys.device)))
    _lib.check(st, "nq_score_keykey_noalloc")
    return out


def keep_plan(seq: int, rate: float, sliding_window: int) -> Tuple[int, int]:
    """(prefix, k) of the keep mask, in Python double as pipeline.py:924-925, 944-946."""
    prefix = max(seq - sliding_window, 0)
    n_keep = max(1, int(prefix * (1.0 - rate)))
    k = min(n_keep, prefix - 1) if (prefix > 1 and n_keep > 0) else 0
    return prefix, max(k, 0)


def keep_mask(importance: torch.Tensor, rate: float, sliding_window: int = 32,
              protected_positions=None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(keep uint8 [b, s], kept_idx int32 [b, s], n_kept int32 [b]) on the device.

    Row b of kept_idx holds its n_kept[b] kept positions ascending, then its
    evicted positions descending."""
    lib = _lib.load()
    _lib.require_device(importance, "importance")
    imp = importance.to(torch.float32).contiguous()
    b, s = imp.shape
    dev = imp.device
    prefix, k = keep_plan(s, rate, sliding_window)
    keep = torch.empty(b, s, dtype=torch.uint8, device=dev)
    kept = torch.empty(b, s, dtype=torch.int32, device=dev)
    n_kept = torch.empty(b, dtype=torch.int32, device=dev)
    prot = None
    n_prot = 0
    if protected_positions is not None:
        pl = [int(p) for p in (protected_positions.tolist() if torch.is_tensor(protected_positions)
                               else protected_positions)]
        if pl:
            prot = torch.tensor(pl, dtype=torch.int32, device=dev)
            n_prot = len(pl)
    with torch.cuda.device(dev):
        st = lib.nq_keep_mask(_addr(imp), b, s, int(sliding_window), prefix, k, _addr(prot), n_prot,
                              _addr(keep), _addr(kept), _addr(n_kept),
                              ctypes.c_void_p(_lib.current_stream_handle(dev)))
    _lib.check(st, "nq_keep_mask")
    return keep, kept, n_kept


def merge_values(values: Sequence[torch.Tensor], keep: torch.Tensor, kept_idx: torch.Tensor,
                 n_kept: torch.Tensor, importance: torch.Tensor, *, centroids: bool = False,
                 survivors: bool = False):
    """Merge eviction over same-shaped value tensors [b, h, s, d] (nq_merge_values).

    keep / kept_idx / n_kept are keep_mask()'s outputs for this seq.  Returns
    (merged tensors, centroids [b, s, d] fp32 or None, survivor [b, s] int32 or
    None: the survivor position of each evicted position, -1 at kept ones).
    """
    lib = _lib.load()
    if not values:
        return [], None, None
    v0 = values[0]
    _lib.require_device(v0, "value tensor")
    if v0.dim() != 4:
        raise ValueError(f"expected value tensors [batch, heads, seq, head_dim], got {tuple(v0.shape)}")
    b, h, s, d = v0.shape
    for v in values:
        if v.shape != v0.shape or v.dtype != v0.dtype or v.device != v0.device:
            raise NotImplementedError("merge eviction over layers of different value shapes or dtypes")
    if d not in (64, 96, 128, 256) or h > 256:
        raise NotImplementedError(f"merge eviction takes head_dim 64, 96, 128 or 256 and <= 256 heads "
                                  f"(got {d}, {h})")
    if tuple(keep.shape) != (b, s) or tuple(kept_idx.shape) != (b, s) or tuple(importance.shape) != (b, s):
        raise ValueError("keep, kept_idx and importance must be [batch, seq]")
    dev = v0.device
    src = [v.contiguous() for v in values]
    src = [v if v.data_ptr() % 16 == 0 else v.clone() for v in src]  # 16-byte vector accesses
    out = list(torch.empty(len(src), b, h, s, d, dtype=v0.dtype, device=dev).unbind(0))
    kp = keep.to(device=dev, dtype=torch.uint8).contiguous()
    ki = kept_idx.to(device=dev, dtype=torch.int32).contiguous()
    nk = n_kept.to(device=dev, dtype=torch.int32).contiguous()
    imp = importance.to(device=dev, dtype=torch.float32).contiguous()
    cent = torch.empty(b, s, d, dtype=torch.float32, device=dev) if centroids else None
    surv = torch.empty(b, s, dtype=torch.int32, device=dev) if survivors else None
    ws_bytes = lib.nq_merge_workspace(b, s, d)
    ws = workspace(dev, ws_bytes)
    staged = _PtrArrays([src, out], dev)
    arrays = staged.arrays
    desc = _lib.MergeDesc(n_tensors=len(src), batch=b, heads=h, seq=s, head_dim=d,
                          dtype=_lib.dtype_code(v0.dtype), src=_addr(arrays[0]), dst=_addr(arrays[1]),
                          keep=_addr(kp), kept_idx=_addr(ki), n_kept=_addr(nk), importance=_addr(imp),
                          centroids=_addr(cent), survivor=_addr(surv), workspace=_addr(ws),
                          workspace_bytes=ws_bytes)
    with torch.cuda.device(dev):
        try:
            st = lib.nq_merge_values(ctypes.byref(desc), ctypes.c_void_p(_lib.current_stream_handle(dev)))
        finally:
            staged.release()
    _lib.check(st, "nq_merge_values")
    return out, cent, surv


def gather_rows(tensors: Sequence[torch.Tensor], *, gather: Optional[torch.Tensor] = None,
                keep: Optional[torch.Tensor] = None) -> List[torch.Tensor]:
    """fp16 passthrough of same-shaped tensors: gathered rows or zeroed evicted rows."""
    lib = _lib.load()
    if not tensors:
        return []
    t0 = tensors[0]
    _lib.require_device(t0, "KV tensor")
    b, h, s, d = t0.shape
    dev = t0.device
    src = [t.contiguous() for t in tensors]
    src = [t if t.data_ptr() % 16 == 0 else t.clone() for t in src]
    g = None
    seq_out = s
    if gather is not None:
        g = gather.to(device=dev, dtype=torch.int32).contiguous()
        if g.dim() == 1:
            g = g.unsqueeze(0).expand(b, -1).contiguous()
        seq_out = g.shape[1]
        if g.numel() and (int(g.min()) < 0 or int(g.max()) >= s):
            raise ValueError(f"gather indices must lie in [0, {s})")
    k = None
    if keep is not None:
        k = keep.to(device=dev, dtype=torch.uint8).contiguous()
        if tuple(k.shape) != (b, s):
            raise ValueError(f"keep must be [batch, seq] = {(b, s)}")
    out = list(torch.empty(len(src), b, h, seq_out, d, dtype=torch.float16, device=dev).unbind(0))
    staged = _PtrArrays([src, out], dev)
    arr_src, arr_dst = staged.arrays
    with torch.cuda.device(dev):
        try:
            st = lib.nq_gather_rows(_addr(arr_src), _addr(arr_dst), len(src), _lib.dtype_code(t0.dtype), b, h, s,
                                    seq_out, d, _addr(g), _addr(k),
                                    ctypes.c_void_p(_lib.current_stream_handle(dev)))
        finally:
            staged.release()
    _lib.check(st, "nq_gather_rows")
    return out
