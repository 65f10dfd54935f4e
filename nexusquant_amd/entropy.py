"""GPU rANS entropy stage for lattice codes (nexusquant/core/entropy_coder.py).

The codes (int8 c = 2p of the relaxed-E8 points, as nq_codes_to_int8 and the
page encoder write them) are histogrammed, coded and decoded on the device by
nq_rans_* (nq_rans.hip).  The coder is the reference's 32-bit / 16-bit-word
rANS with 12-bit probabilities; the stream is cut into chunks that are coded
independently (one lane each), so each chunk's words equal the reference
encoder's output for that chunk.  The frequency table follows the reference's
normalisation rule exactly (build_freq_table), computed on the host from the
device histogram (at most 33 entries).

NQR1 container (little endian):
    b"NQR1", u16 version = 1, u8 levels, u8 has_half, u16 alphabet, u16 pad,
    u64 n_symbols, u32 chunk, u32 n_chunks, u16 freq[alphabet] (padded to 4 bytes),
    u64 offsets[n_chunks + 1] (in 16-bit words), u16 words[offsets[-1]],
    then an optional fp32 scale section: u64 n_scales, f32 scales[n_scales].
The reference's encode_e8 writes one stream with fp16 scales; NQR1 keeps the
fp32 scales (lossless) and the chunk offsets that make decoding parallel.

The reference's own container is written and read by encode_e8 / decode_e8
below (entropy_coder.py:360-431): header '<IBBI' (n_groups, levels, has_half,
n_symbols), lengths '<III', u16 alphabet + u16 freq[alphabet], fp16 scales,
then the u16 words of ONE rANS stream over all symbols.  That stream is a
single dependency chain, coded here by one GPU lane (the chunked coder with one
chunk spanning the stream), so it runs at the chain's latency (about 80 ns a
symbol); NQR1 is the parallel format.
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
import struct
from typing import Optional

import numpy as np
import torch

from . import _lib
from .ops import _addr

PROB_BITS = 12
M = 1 << PROB_BITS
# symbols per chunk at most (nq_rans_encode / nq_rans_decode take an int32 chunk)
MAX_CHUNK = (1 << 31) - 1
DEFAULT_CHUNK = 2048  # symbols per chunk (one lane's chain); see the measurements in the design notes
_MAGIC = b"NQR1"


def build_freq_table(counts: np.ndarray) -> np.ndarray:
    """Frequencies summing to 4096 from symbol counts, by the reference's rule
    (entropy_coder.py:175-243): every seen symbol gets 1, the rest is shared in
    proportion to the counts (floored), leftovers go to the largest fractional
    parts, an excess is taken back from the rarest symbols."""
    counts = np.asarray(counts, dtype=np.int64)
    alphabet = len(counts)
    total = counts.sum()
    if total == 0:
        freqs = np.ones(alphabet, dtype=np.int64) * (M // alphabet)
        freqs[0] += M - freqs.sum()
    else:
        seen = counts > 0
        n_seen = int(seen.sum())
        freqs = np.zeros(alphabet, dtype=np.int64)
        freqs[seen] = 1
        remaining = M - n_seen
        if remaining > 0:
            prop = (counts[seen].astype(np.float64) / total) * remaining
            extra = np.floor(prop).astype(np.int64)
            freqs[seen] += extra
            diff = int(M - freqs.sum())
            seen_idx = np.where(seen)[0]
            if diff > 0:
                order = seen_idx[np.argsort(-(prop - extra))]
                for i in range(diff):
                    freqs[order[i % len(order)]] += 1
            elif diff < 0:
                order = seen_idx[np.argsort(counts[seen])]
                removed = 0
                for idx in order:
                    while freqs[idx] > 1 and removed < -diff:
                        freqs[idx] -= 1
                        removed += 1
                    if removed >= -diff:
                        break
        elif remaining < 0:
            seen_idx = np.where(seen)[0]
            order = seen_idx[np.argsort(-counts[seen])]
            freqs[:] = 0
            for i in range(min(M, len(order))):
                freqs[order[i]] = 1
    if freqs.sum() != M:
        raise AssertionError(f"frequency table sums to {freqs.sum()}, not {M}")
    return freqs.astype(np.uint16)


@dataclasses.dataclass
class RansStream:
    """Device-resident chunked rANS stream of n int8 codes."""
    words: torch.Tensor     # int16 view of the uint16 words
    offsets: torch.Tensor   # int64 [n_chunks + 1]
    freq: np.ndarray        # uint16 [alphabet]
    levels: int
    has_half: bool
    n: int
    chunk: int
    shape: tuple
    # layout key of the state last checked against the decoder's bounds (set by
    # rans_encode, unpack_nqr1 and rans_decode); any reassignment or in-place
    # change of words, offsets or freq makes it stale
    _checked: Optional[tuple] = dataclasses.field(default=None, repr=False, compare=False)

    @property
    def alphabet(self) -> int:
        return len(self.freq)

    def _layout_key(self) -> tuple:
        return (id(self.words), self.words._version, id(self.offsets), self.offsets._version, self.levels,
                bool(self.has_half), self.n, self.chunk, self.freq.tobytes(), self.words.numel(),
                self.offsets.numel())

    def nbytes(self) -> int:
        """Coded size: words, chunk offsets and the frequency table."""
        return 2 * self.words.numel() + 8 * self.offsets.numel() + 2 * self.alphabet


def _stream(dev) -> ctypes.c_void_p:
    return ctypes.c_void_p(_lib.current_stream_handle(dev))


# codes per histogram call: the kernel's bins are 32-bit, read here as int32,
# so every piece keeps each bin below 2^31; the pieces are summed in int64
_HIST_PIECE = 1 << 30


def _code_counts(flat: torch.Tensor, levels: int) -> np.ndarray:
    """Histogram of c + levels over the 2 * levels + 1 codes (device passes).

    flat is 16-byte aligned; so is every piece, at multiples of 2^30 codes."""
    lib = _lib.load()
    dev = flat.device
    n = flat.numel()
    total = torch.zeros(2 * levels + 1, dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        for start in range(0, n, _HIST_PIECE):
            piece = flat[start:start + _HIST_PIECE]
            hist = torch.zeros(2 * levels + 1, dtype=torch.int32, device=dev)
            _lib.check(lib.nq_rans_histogram(_addr(piece), piece.numel(), levels, _addr(hist), _stream(dev)),
                       "nq_rans_histogram")
            total += hist.to(torch.int64)
    return total.cpu().numpy()


def rans_encode(codes: torch.Tensor, levels: int, chunk: int = DEFAULT_CHUNK,
                has_half: Optional[bool] = None) -> RansStream:
    """rANS-code int8 codes c = 2p (|c| <= levels) on the device.

    has_half (default: some code is odd) selects the alphabet: c + levels over
    2 * levels + 1 symbols, else c / 2 + levels / 2 over levels + 1."""
    lib = _lib.load()
    _lib.require_device(codes, "codes")
    if codes.dtype != torch.int8:
        raise TypeError(f"codes must be int8 (2p), got {codes.dtype}")
    if levels not in (2, 4, 8, 16):
        raise ValueError(f"levels must be 2, 4, 8 or 16, got {levels}")
    dev = codes.device
    flat = codes.contiguous().reshape(-1)
    if flat.data_ptr() % 16:
        flat = flat.clone()
    n = flat.numel()
    h = _code_counts(flat, levels)
    if has_half is None:
        # odd bins hold the half-integer codes (c + L odd <=> c odd for even L)
        has_half = bool(h[1::2].sum() > 0)
    elif not has_half and h[1::2].sum() > 0:
        raise ValueError("has_half=False but some codes are odd (half-integer points)")
    counts = h if has_half else h[0::2]
    freq = build_freq_table(counts)
    alphabet = len(freq)
    n_chunks = (n + chunk - 1) // chunk
    freq_d = torch.from_numpy(freq.view(np.int16).copy()).to(dev)
    scratch = torch.empty(max(int(lib.nq_rans_scratch_words(n, chunk)), 1), dtype=torch.int16, device=dev)
    n_words = torch.empty(max(n_chunks, 1), dtype=torch.int32, device=dev)
    offsets = torch.empty(n_chunks + 1, dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.nq_rans_encode(_addr(flat), n, levels, int(has_half), _addr(freq_d), alphabet, chunk,
                                      _addr(scratch), _addr(n_words), _addr(offsets), _stream(dev)),
                   "nq_rans_encode")
        total = int(offsets[-1].item())
        words = torch.empty(max(total, 1), dtype=torch.int16, device=dev)
        _lib.check(lib.nq_rans_compact(_addr(scratch), _addr(n_words), _addr(offsets), n, chunk, _addr(words),
                                       _stream(dev)), "nq_rans_compact")
    st = RansStream(words=words[:total], offsets=offsets, freq=freq, levels=levels, has_half=has_half, n=n,
                    chunk=chunk, shape=tuple(codes.shape))
    st._checked = st._layout_key()  # offsets written by nq_rans_encode's scan: consistent by construction
    return st


# Batched coding of many tensors (one stream each, e.g. one per layer and role).
# One tensor's stream at the default chunk has 65536 chains, one wave per SIMD,
# so a single launch leaves most of each SIMD idle and a loop of calls runs them
# one after another with two host round trips each.  The batched calls run the
# launches of different tensors on worker streams at once and pipeline groups
# of tensors: while a group's encoder launches run on the workers, the next
# group's histograms run on the caller's stream, and one host round trip reads
# both the group's word totals and the next group's histograms.  The streams
# are the ones rans_encode writes, word for word.
_WORKER_STREAMS = 3   # with the caller's stream, the 4 hardware queues a process gets here
_BATCH_GROUP = 16     # tensors per group (bounds the scratch memory in flight)
_workers = {}


def _worker_streams(dev) -> list:
    key = torch.device(dev).index
    if key not in _workers:
        _workers[key] = [torch.cuda.Stream(device=dev) for _ in range(_WORKER_STREAMS)]
    return _workers[key]


def _prepare_codes(codes: torch.Tensor, levels: int) -> torch.Tensor:
    _lib.require_device(codes, "codes")
    if codes.dtype != torch.int8:
        raise TypeError(f"codes must be int8 (2p), got {codes.dtype}")
    if levels not in (2, 4, 8, 16):
        raise ValueError(f"levels must be 2, 4, 8 or 16, got {levels}")
    flat = codes.contiguous().reshape(-1)
    if flat.data_ptr() % 16:
        flat = flat.clone()
    return flat


def rans_encode_many(codes_list, levels, chunk: int = DEFAULT_CHUNK, has_half=None) -> list:
    """rans_encode of each tensor of codes_list (levels / has_half: one value for
    all, or one per tensor), the launches of different tensors overlapping on a
    few worker streams.  Returns the RansStreams rans_encode would return; the
    words and offsets of the streams of one group of tensors are views of one
    buffer each, which lives while any of them does."""
    lib = _lib.load()
    n_t = len(codes_list)
    lv = list(levels) if isinstance(levels, (list, tuple)) else [levels] * n_t
    hh = list(has_half) if isinstance(has_half, (list, tuple)) else [has_half] * n_t
    if len(lv) != n_t or len(hh) != n_t:
        raise ValueError("levels and has_half take one value or one per tensor")
    if n_t == 0:
        return []
    flats = [_prepare_codes(c, l) for c, l in zip(codes_list, lv)]
    if len({f.device for f in flats}) != 1:
        raise ValueError("rans_encode_many: all tensors must be on one device")
    dev = flats[0].device
    groups = [list(range(g, min(n_t, g + _BATCH_GROUP))) for g in range(0, n_t, _BATCH_GROUP)]
    out = []
    with torch.cuda.device(dev):
        cur = torch.cuda.current_stream(dev)
        h_cur = ctypes.c_void_p(cur.cuda_stream)
        workers = _worker_streams(dev)

        def launch_hists(idx):  # int64 [len(idx), 33] on the caller's stream
            tot = torch.zeros(len(idx), 33, dtype=torch.int64, device=dev)
            for r, i in enumerate(idx):
                bins = 2 * lv[i] + 1
                for start in range(0, flats[i].numel(), _HIST_PIECE):
                    piece = flats[i][start:start + _HIST_PIECE]
                    hist = torch.zeros(bins, dtype=torch.int32, device=dev)
                    _lib.check(lib.nq_rans_histogram(_addr(piece), piece.numel(), lv[i], _addr(hist), h_cur),
                               "nq_rans_histogram")
                    tot[r, :bins] += hist.to(torch.int64)
            return tot

        counts = launch_hists(groups[0]).cpu().numpy()
        for gi, idx in enumerate(groups):
            plans = []
            for r, i in enumerate(idx):
                h = counts[r, :2 * lv[i] + 1]
                half = hh[i]
                if half is None:
                    half = bool(h[1::2].sum() > 0)
                elif not half and h[1::2].sum() > 0:
                    raise ValueError("has_half=False but some codes are odd (half-integer points)")
                freq = build_freq_table(h if half else h[0::2])
                n = flats[i].numel()
                plans.append(dict(flat=flats[i], n=n, levels=lv[i], half=half, freq=freq,
                                  n_chunks=(n + chunk - 1) // chunk, shape=tuple(codes_list[i].shape)))
            freq_all = torch.from_numpy(np.concatenate([p["freq"].view(np.int16) for p in plans]).copy()).to(dev)
            # one allocation per group for each kind of buffer, sliced per tensor;
            # scratch slices start on 8-byte boundaries (4-word multiples)
            sw = [(max(int(lib.nq_rans_scratch_words(p["n"], chunk)), 1) + 3) // 4 * 4 for p in plans]
            scratch_all = torch.empty(sum(sw), dtype=torch.int16, device=dev)
            nw_all = torch.empty(sum(max(p["n_chunks"], 1) for p in plans), dtype=torch.int32, device=dev)
            off_all = torch.empty(sum(p["n_chunks"] + 1 for p in plans), dtype=torch.int64, device=dev)
            base = bs = bn = bo = 0
            for p, w in zip(plans, sw):
                p["freq_d"] = freq_all[base:base + len(p["freq"])]
                base += len(p["freq"])
                p["scratch"] = scratch_all[bs:bs + w]
                bs += w
                p["n_words"] = nw_all[bn:bn + max(p["n_chunks"], 1)]
                bn += max(p["n_chunks"], 1)
                p["offsets"] = off_all[bo:bo + p["n_chunks"] + 1]
                bo += p["n_chunks"] + 1
            ready = cur.record_event()
            for w in workers:
                w.wait_event(ready)
            for k, p in enumerate(plans):
                s = workers[k % len(workers)]
                _lib.check(lib.nq_rans_encode(_addr(p["flat"]), p["n"], p["levels"], int(p["half"]), _addr(p["freq_d"]),
                                              len(p["freq"]), chunk, _addr(p["scratch"]), _addr(p["n_words"]),
                                              _addr(p["offsets"]), ctypes.c_void_p(s.cuda_stream)), "nq_rans_encode")
            # the next group's histograms run beside this group's encoders
            nxt = launch_hists(groups[gi + 1]) if gi + 1 < len(groups) else None
            for w in workers:
                cur.wait_stream(w)
            totals = torch.stack([p["offsets"][-1] for p in plans])
            if nxt is not None:
                both = torch.cat([totals, nxt.reshape(-1)]).cpu().numpy()
                totals_h, counts = both[:len(plans)], both[len(plans):].reshape(-1, 33)
            else:
                totals_h = totals.cpu().numpy()
            ww = [(max(int(t), 1) + 3) // 4 * 4 for t in totals_h]  # 8-byte aligned slices
            words_all = torch.empty(sum(ww), dtype=torch.int16, device=dev)
            bw = 0
            for p, total, w in zip(plans, totals_h, ww):
                p["total"] = int(total)
                p["words"] = words_all[bw:bw + w]
                bw += w
            ready = cur.record_event()
            for w in workers:
                w.wait_event(ready)
            for k, p in enumerate(plans):
                s = workers[k % len(workers)]
                _lib.check(lib.nq_rans_compact(_addr(p["scratch"]), _addr(p["n_words"]), _addr(p["offsets"]), p["n"],
                                               chunk, _addr(p["words"]), ctypes.c_void_p(s.cuda_stream)),
                           "nq_rans_compact")
            # the caller's stream waits for the compactions, so the scratch buffers
            # (allocated on it) are reused only after them
            for w in workers:
                cur.wait_stream(w)
            for p in plans:
                st = RansStream(words=p["words"][:p["total"]], offsets=p["offsets"], freq=p["freq"], levels=p["levels"],
                                has_half=p["half"], n=p["n"], chunk=chunk, shape=p["shape"])
                st._checked = st._layout_key()
                out.append(st)
    return out


def rans_decode_many(streams, device=None) -> list:
    """rans_decode of each stream, the launches overlapping on a few worker
    streams; returns the int8 codes in each stream's shape."""
    lib = _lib.load()
    outs, jobs = [], []
    for stream in streams:
        key = stream._layout_key()
        if stream._checked != key:
            check_stream_layout(stream.levels, stream.has_half, stream.alphabet, stream.n, stream.chunk,
                                stream.offsets.numel() - 1, stream.freq, stream.offsets.cpu().numpy(),
                                stream.words.numel())
            stream._checked = key
        if int(np.prod(stream.shape)) != stream.n:
            raise ValueError(f"stream shape {stream.shape} does not hold {stream.n} symbols")
        dev = stream.words.device if device is None else torch.device(device)
        out = torch.empty(stream.n, dtype=torch.int8, device=dev)
        outs.append(out.reshape(stream.shape))
        if stream.n:
            words = stream.words.to(dev)
            if words.numel() == 0:
                words = torch.zeros(1, dtype=torch.int16, device=dev)
            if words.data_ptr() % 8:
                words = words.clone()
            jobs.append((dev, stream, words, stream.offsets.to(dev), out))
    by_dev = {}
    for job in jobs:
        by_dev.setdefault(job[0], []).append(job)
    for dev, dev_jobs in by_dev.items():
        with torch.cuda.device(dev):
            cur = torch.cuda.current_stream(dev)
            freq_all = torch.from_numpy(np.concatenate([j[1].freq.view(np.int16) for j in dev_jobs]).copy()).to(dev)
            workers = _worker_streams(dev)
            ready = cur.record_event()
            for w in workers:
                w.wait_event(ready)
            base = 0
            keep = []
            for k, (_, stream, words, offsets, out) in enumerate(dev_jobs):
                freq_d = freq_all[base:base + stream.alphabet]
                base += stream.alphabet
                s = workers[k % len(workers)]
                _lib.check(lib.nq_rans_decode(_addr(words), _addr(offsets), stream.n, stream.levels,
                                              int(stream.has_half), _addr(freq_d), stream.alphabet, stream.chunk,
                                              _addr(out), ctypes.c_void_p(s.cuda_stream)), "nq_rans_decode")
                keep.append((words, offsets))
            for w in workers:
                cur.wait_stream(w)  # inputs copied or cloned above are released after this point
            del keep
    return outs


def check_stream_header(levels: int, has_half: bool, alphabet: int, n: int, chunk: int, n_chunks: int) -> None:
    """Raise ValueError unless a stream header's counts agree with each other."""
    if levels not in (2, 4, 8, 16):
        raise ValueError(f"stream levels must be 2, 4, 8 or 16, got {levels}")
    want_alpha = 2 * levels + 1 if has_half else levels + 1
    if alphabet != want_alpha:
        raise ValueError(f"alphabet {alphabet} does not match levels {levels} "
                         f"({'with' if has_half else 'without'} half-integer points: {want_alpha})")
    if chunk < 1 or chunk > MAX_CHUNK:
        raise ValueError(f"chunk must be in [1, 2^31 - 1], got {chunk}")
    if n < 0:
        raise ValueError(f"negative symbol count {n}")
    if n_chunks != (n + chunk - 1) // chunk:
        raise ValueError(f"{n_chunks} chunks for {n} symbols of chunk {chunk}; expected {(n + chunk - 1) // chunk}")


def check_stream_layout(levels: int, has_half: bool, alphabet: int, n: int, chunk: int, n_chunks: int,
                        freq: np.ndarray, offsets: np.ndarray, n_words: int) -> None:
    """Raise ValueError unless a stream's header, frequency table and chunk
    offsets are consistent with each other and with the n_words words present.

    nq_rans_decode recomputes the chunk count as ceil(n / chunk) and reads
    offsets[k] .. offsets[k + 1] of every chunk, and its slot tables are only
    complete when the frequencies sum to 4096, so all of this is checked on
    the host before anything reaches the device."""
    check_stream_header(levels, has_half, alphabet, n, chunk, n_chunks)
    freq = np.asarray(freq)
    if freq.size != alphabet or int(freq.astype(np.int64).sum()) != M:
        raise ValueError(f"frequency table must hold {alphabet} entries summing to {M}")
    offsets = np.asarray(offsets, dtype=np.int64)
    if offsets.size != n_chunks + 1 or (offsets.size and offsets[0] != 0):
        raise ValueError("chunk offsets must hold n_chunks + 1 entries starting at 0")
    if offsets.size > 1:
        per = np.diff(offsets)
        if np.any(per < 0):
            raise ValueError("chunk offsets must be non-decreasing")
        lens = np.full(n_chunks, chunk, dtype=np.int64)
        lens[-1] = n - chunk * (n_chunks - 1)
        if np.any(per > lens + 2):  # a chunk holds its final state plus at most one word per symbol
            raise ValueError("a chunk claims more words than its symbols can produce")
    if offsets.size and int(offsets[-1]) != n_words:
        raise ValueError(f"chunk offsets end at word {int(offsets[-1])} but the stream holds {n_words} words")


def rans_decode(stream: RansStream, device=None) -> torch.Tensor:
    """int8 codes of a RansStream, in its original shape."""
    lib = _lib.load()
    key = stream._layout_key()
    if stream._checked != key:
        check_stream_layout(stream.levels, stream.has_half, stream.alphabet, stream.n, stream.chunk,
                            stream.offsets.numel() - 1, stream.freq, stream.offsets.cpu().numpy(),
                            stream.words.numel())
        stream._checked = key
    if int(np.prod(stream.shape)) != stream.n:
        raise ValueError(f"stream shape {stream.shape} does not hold {stream.n} symbols")
    dev = stream.words.device if device is None else torch.device(device)
    out = torch.empty(stream.n, dtype=torch.int8, device=dev)
    if stream.n:
        words = stream.words.to(dev)
        if words.numel() == 0:
            words = torch.zeros(1, dtype=torch.int16, device=dev)
        if words.data_ptr() % 8:  # the kernel reads 4 words at a time
            words = words.clone()
        offsets = stream.offsets.to(dev)
        freq_d = torch.from_numpy(stream.freq.view(np.int16).copy()).to(dev)
        with torch.cuda.device(dev):
            _lib.check(lib.nq_rans_decode(_addr(words), _addr(offsets), stream.n, stream.levels, int(stream.has_half),
                                          _addr(freq_d), stream.alphabet, stream.chunk, _addr(out), _stream(dev)),
                       "nq_rans_decode")
    return out.reshape(stream.shape)


def pack_nqr1(stream: RansStream, scales: Optional[torch.Tensor] = None) -> bytes:
    """NQR1 bytes of a stream (and optional fp32 scales)."""
    freq = stream.freq.astype("<u2").tobytes()
    freq += b"\0" * ((-len(freq)) % 4)
    n_chunks = stream.offsets.numel() - 1
    head = _MAGIC + struct.pack("<HBBHHQII", 1, stream.levels, int(stream.has_half), stream.alphabet, 0,
                                stream.n, stream.chunk, n_chunks)
    body = stream.offsets.cpu().numpy().astype("<u8").tobytes() + stream.words.cpu().numpy().view("<u2").tobytes()
    tail = b""
    if scales is not None:
        sc = scales.detach().float().cpu().numpy().reshape(-1).astype("<f4")
        tail = struct.pack("<Q", sc.size) + sc.tobytes()
    return head + freq + body + tail


def unpack_nqr1(blob: bytes, shape=None, device="cuda"):
    """(RansStream on `device`, fp32 scales or None) from NQR1 bytes.

    Every length, count and offset is checked against the blob before any
    array is built (ValueError on a truncated or inconsistent container)."""
    head = 4 + struct.calcsize("<HBBHHQII")
    if len(blob) < head or blob[:4] != _MAGIC:
        raise ValueError("not an NQR1 stream")
    version, levels, has_half, alphabet, _, n, chunk, n_chunks = struct.unpack_from("<HBBHHQII", blob, 4)
    if version != 1:
        raise ValueError(f"NQR1 version {version} unsupported")
    check_stream_header(levels, bool(has_half), alphabet, n, chunk, n_chunks)
    at = head

    def need(nbytes, what):
        if nbytes < 0 or at + nbytes > len(blob):
            raise ValueError(f"truncated NQR1 stream: {what} needs {nbytes} bytes at offset {at}, "
                             f"{len(blob)} bytes in the blob")

    need(2 * alphabet, "frequency table")
    freq = np.frombuffer(blob, dtype="<u2", count=alphabet, offset=at).astype(np.uint16)
    at += 2 * alphabet + ((-2 * alphabet) % 4)
    need(8 * (n_chunks + 1), "chunk offsets")
    offsets = np.frombuffer(blob, dtype="<u8", count=n_chunks + 1, offset=at).astype(np.int64)
    at += 8 * (n_chunks + 1)
    n_words = int(offsets[-1])
    need(2 * n_words, "words")
    check_stream_layout(levels, bool(has_half), alphabet, n, chunk, n_chunks, freq, offsets, n_words)
    if shape is not None and int(np.prod(shape)) != n:
        raise ValueError(f"shape {tuple(shape)} does not hold the stream's {n} symbols")
    words = np.frombuffer(blob, dtype="<u2", count=n_words, offset=at).view(np.int16)
    at += 2 * n_words
    scales = None
    if at < len(blob):
        need(8, "scale count")
        (ns,) = struct.unpack_from("<Q", blob, at)
        at += 8
        need(4 * ns, "scales")
        if at + 4 * ns != len(blob):
            raise ValueError(f"{len(blob) - at - 4 * ns} trailing bytes after the NQR1 scales")
        scales = torch.from_numpy(np.frombuffer(blob, dtype="<f4", count=ns, offset=at).copy())
    dev = torch.device(device)
    stream = RansStream(words=torch.from_numpy(words.copy()).to(dev), offsets=torch.from_numpy(offsets.copy()).to(dev),
                        freq=freq, levels=levels, has_half=bool(has_half), n=n, chunk=chunk,
                        shape=tuple(shape) if shape is not None else (n,))
    stream._checked = stream._layout_key()  # checked above against the blob
    return stream, scales


def shannon_bits(counts: np.ndarray) -> float:
    """Total Shannon information of a symbol histogram, in bits."""
    c = np.asarray(counts, dtype=np.float64)
    c = c[c > 0]
    if c.size == 0:
        return 0.0
    p = c / c.sum()
    return float(-(c * np.log2(p)).sum())


# ---------------------------------------------------------------------------
# The reference's single-stream container: encode_e8 / decode_e8
# ---------------------------------------------------------------------------

E8_HEADER = struct.Struct("<IBBI")    # n_groups, levels, has_half, n_symbols (entropy_coder.py:406-408)
E8_LENGTHS = struct.Struct("<III")    # freq, scale and rANS section lengths in bytes (:421-424)


def _e8_codes(quantized: torch.Tensor, scale_factors: torch.Tensor, levels: int):
    """(codes int8 [n], has_half, device fp32 scales) of encode_e8's symbol step."""
    lib = _lib.load()
    _lib.require_device(quantized, "quantized")
    if levels not in (2, 4, 8, 16):
        raise ValueError(f"levels must be 2, 4, 8 or 16, got {levels}")
    if quantized.numel() % 8:
        raise RuntimeError(f"shape '[-1, 8]' is invalid for input of size {quantized.numel()}")
    dev = quantized.device
    flat = quantized.reshape(-1, 8).float().contiguous()
    if flat.data_ptr() % 16:
        flat = flat.clone()
    scales = scale_factors.reshape(-1).float().to(dev).contiguous()
    n_groups, n_scales = flat.shape[0], scales.numel()
    if n_scales not in (1, n_groups):
        raise ValueError(f"operands could not be broadcast together: {n_groups} groups of 8 and {n_scales} "
                         "scale factors")
    codes = torch.empty(n_groups * 8, dtype=torch.int8, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.nq_e8_stream_codes(_addr(flat), _addr(scales), n_groups, n_scales, levels, _addr(codes),
                                          _addr(flag), _stream(dev)), "nq_e8_stream_codes")
    return codes, bool(flag.item()), scales


def encode_e8(quantized: torch.Tensor, scale_factors: torch.Tensor, levels: int = 8) -> bytes:
    """The reference's rANS container of an E8-quantized tensor (entropy_coder.py:360-426).

    quantized: scaled lattice points on a ROCm device (any shape, groups of 8);
    scale_factors: one per group of 8, or one in all.  The bytes equal the
    reference's for the same inputs.  The container codes every symbol in one
    rANS chain; this build takes up to 2^31 - 1 symbols per container."""
    if quantized.numel() > MAX_CHUNK:
        raise ValueError(f"encode_e8 codes all symbols as one rANS chain; this build takes at most 2^31 - 1 "
                         f"symbols per container, got {quantized.numel()} (encode the tensor in pieces)")
    codes, has_half, scales = _e8_codes(quantized, scale_factors, levels)
    n = codes.numel()
    if n:
        st = rans_encode(codes, levels, chunk=n, has_half=has_half)
        freq, words = st.freq, st.words.cpu().numpy().view("<u2")
    else:
        # no symbols: the table of an empty histogram, and the initial state
        # 2^16 flushed as two words
        freq = build_freq_table(np.zeros(levels + 1, np.int64))
        words = np.array([1, 0], dtype="<u2")
    freq_bytes = struct.pack("<H", len(freq)) + freq.astype("<u2").tobytes()
    scale_f16 = scales.clamp_min(1e-8).half().cpu().numpy().astype("<f2").tobytes()
    rans = words.astype("<u2").tobytes()
    return (E8_HEADER.pack(n // 8, levels, int(has_half), n) + E8_LENGTHS.pack(len(freq_bytes), len(scale_f16),
                                                                               len(rans))
            + freq_bytes + scale_f16 + rans)


def decode_e8(compressed: bytes, original_shape: Optional[tuple] = None, device=None):
    """(quantized fp32, scales fp32) of an encode_e8 container (entropy_coder.py:429-475).

    Decoding runs on the GPU (the current device unless `device` is given);
    the results come back on the host, as the reference returns them, unless
    `device` is given."""
    lib = _lib.load()
    n_groups, levels, has_half, n_symbols = E8_HEADER.unpack_from(compressed, 0)
    at = E8_HEADER.size
    freq_len, scale_len, rans_len = E8_LENGTHS.unpack_from(compressed, at)
    at += E8_LENGTHS.size
    if at + freq_len + scale_len + rans_len > len(compressed):
        raise ValueError(f"truncated E8 stream: sections of {freq_len}, {scale_len} and {rans_len} bytes "
                         f"after a {at}-byte header, {len(compressed)} bytes in all")
    if freq_len < 2:
        raise ValueError("E8 stream without a frequency table")
    (alphabet,) = struct.unpack_from("<H", compressed, at)
    if 2 + 2 * alphabet > freq_len:
        raise ValueError(f"frequency table of {alphabet} entries does not fit its {freq_len} bytes")
    freq = np.frombuffer(compressed, dtype="<u2", count=alphabet, offset=at + 2).astype(np.uint16)
    at += freq_len
    scales_f16 = np.frombuffer(compressed, dtype="<f2", count=scale_len // 2, offset=at).copy()
    at += scale_len
    words = np.frombuffer(compressed, dtype="<u2", count=rans_len // 2, offset=at).copy()
    if n_symbols != 8 * n_groups:
        raise ValueError(f"cannot reshape {n_symbols} symbols into {n_groups} groups of 8")
    if n_symbols > MAX_CHUNK:
        raise ValueError(f"decode_e8 decodes one rANS chain of at most 2^31 - 1 symbols in this build; the "
                         f"container holds {n_symbols}")
    n_scales = scales_f16.size
    if n_scales not in (1, n_groups) and n_groups:
        raise ValueError(f"operands could not be broadcast together: {n_groups} groups of 8 and {n_scales} scales")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(n_groups, 8, dtype=torch.float32, device=dev)
    if n_symbols:
        stream = RansStream(words=torch.from_numpy(words.view(np.int16)).to(dev),
                            offsets=torch.tensor([0, words.size], dtype=torch.int64, device=dev),
                            freq=freq, levels=levels, has_half=bool(has_half), n=n_symbols, chunk=n_symbols,
                            shape=(n_symbols,))
        codes = rans_decode(stream)
        sc = torch.from_numpy(scales_f16.view(np.int16)).to(dev)
        with torch.cuda.device(dev):
            _lib.check(lib.nq_e8_stream_values(_addr(codes), _addr(sc), n_groups, n_scales, _addr(out),
                                               _stream(dev)), "nq_e8_stream_values")
    scales = torch.from_numpy(scales_f16.astype(np.float32))
    if original_shape is not None:
        out = out.reshape(original_shape)
    if device is None:
        return out.cpu(), scales
    return out, scales.to(dev)


def measure_entropy(indices, alphabet_size: Optional[int] = None) -> dict:
    """Shannon entropy statistics of a symbol stream (entropy_coder.py:94-133)."""
    if torch.is_tensor(indices):
        counts = torch.bincount(indices.reshape(-1).long()).cpu().numpy()
        unique = np.nonzero(counts)[0]
        counts = counts[unique]
    else:
        unique, counts = np.unique(np.asarray(indices), return_counts=True)
    return _entropy_from_counts(unique, counts, alphabet_size)


def _entropy_from_counts(unique: np.ndarray, counts: np.ndarray, alphabet_size: Optional[int]) -> dict:
    n = int(np.sum(counts))
    if n == 0:
        return {"entropy_bps": 0, "uniform_bps": 0, "compression_ratio": 1.0, "n_symbols": 0, "n_unique": 0}
    probs = counts / n
    entropy = -np.sum(probs * np.log2(probs + 1e-30))
    if alphabet_size is None:
        alphabet_size = int(unique.max()) + 1
    uniform_bps = math.log2(max(alphabet_size, 2))
    return {"entropy_bps": float(entropy), "uniform_bps": float(uniform_bps),
            "compression_ratio": float(uniform_bps / max(entropy, 0.01)), "n_symbols": int(n),
            "n_unique": int(len(unique))}


def _symbol_stats(codes: torch.Tensor, levels: int, has_half: bool) -> dict:
    h = _code_counts(codes, levels)
    counts = h if has_half else h[0::2]
    unique = np.nonzero(counts)[0]
    return _entropy_from_counts(unique, counts[unique], len(counts))


def measure_e8_entropy(quantized: torch.Tensor, scale_factors: torch.Tensor, levels: int = 8) -> dict:
    """Entropy statistics of the symbols encode_e8 would code (entropy_coder.py:136-157)."""
    codes, has_half, _ = _e8_codes(quantized, scale_factors, levels)
    return _symbol_stats(codes, levels, has_half)


def e8_quantize_with_entropy(x: torch.Tensor, levels: int = 8, return_stats: bool = True) -> dict:
    """Per-8-group E8 quantization, encode_e8 and decode_e8 with the size
    accounting of entropy_coder.py:478-570.  Tensors stay on x's device."""
    from .kernels import e8_quantize_perhead
    _lib.require_device(x, "x")
    shape = x.shape
    pad = (8 - shape[-1] % 8) % 8
    x_padded = torch.nn.functional.pad(x, (0, pad)) if pad else x
    flat = x_padded.reshape(-1, 8).float()
    # per-group scale: the per-row rule on rows of 8 (amax clamped to 1e-8, / (levels / 2))
    sc = flat.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8) / (levels / 2)
    quantized_scaled = e8_quantize_perhead(flat, levels)
    compressed = encode_e8(quantized_scaled, sc, levels=levels)
    decoded, _ = decode_e8(compressed, original_shape=flat.shape, device=x.device)
    reconstructed = decoded.reshape(x_padded.shape)
    if pad:
        reconstructed = reconstructed[..., :shape[-1]]
    reconstructed = reconstructed.reshape(shape)
    n_coords, n_groups = flat.numel(), flat.shape[0]
    n_bytes_uniform = math.ceil(n_coords * math.ceil(math.log2(levels + 1)) / 8) + n_groups * 2
    n_bytes_compressed = len(compressed)
    original_bytes = n_coords * 2
    result = {
        "compressed_bytes": compressed,
        "reconstructed": reconstructed,
        "scale_factors": sc,
        "n_bytes_compressed": n_bytes_compressed,
        "n_bytes_uniform": n_bytes_uniform,
        "n_bytes_original": original_bytes,
        "rans_compression_ratio": n_bytes_uniform / max(n_bytes_compressed, 1),
        "e8_base_ratio": original_bytes / n_bytes_uniform,
        "total_compression_ratio": original_bytes / n_bytes_compressed,
    }
    if return_stats:
        codes, has_half, _ = _e8_codes(quantized_scaled, sc, levels)
        result["entropy_stats"] = _symbol_stats(codes, levels, has_half)
    return result
