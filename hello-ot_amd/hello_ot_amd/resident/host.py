"""One side of the problem kept in host memory and streamed to the device in row chunks.

This is the reference's resident / streamed split (``kernels/bilinear_topk.py:99-118, 255-368``,
``kernels/scan_contract.py:113-253``): one side stays on the device, the other is read in bounded chunks, so the
device holds one side's features plus O(chunk * d) of staging instead of both sides. Here the streamed side's rows
stay in the caller's host tensor and pass, in the solver's shuffled order, through two pinned staging buffers of one
chunk each (bounded pinned memory, as in the reference): the host gathers chunk c into a staging buffer once that
buffer's previous upload has finished, a side stream of default priority uploads it into one of two device buffers
once the work queued on that buffer's previous chunk has finished, and the caller's stream waits for the upload.
Host copies and uploads of the next chunk run on a worker thread while the caller works on the current one.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import torch

# fp32 features per streamed chunk: 19968 rows at d = 8192, the internal chunk the l2^2 scan itself takes for
# 1.28M columns (78 panels of 256 rows, whose column lists of k = 16 fill its 12 GiB list budget), so a streamed scan
# finalizes its columns as often as a one-call scan
STREAM_CHUNK_BYTES = 78 * 256 * 8192 * 4
STREAM_MIN_BYTES = 4 << 30       # a side (or a level's prefix of it) smaller than this is copied to the device whole
# Where the source side lives when the caller does not ask for both sides on the device: "auto" streams it when the
# resident plan would need more than RESIDENT_BUDGET of the device's memory, "always" streams every source side
# above STREAM_MIN_BYTES, "never" keeps it resident. The environment variable HELLOOT_STREAM_SOURCE overrides it.
STREAM_POLICY = "auto"
RESIDENT_BUDGET = 0.75


class HostRows:
    """Rows of a host fp32 matrix, read by the device in chunks of at most ``chunk`` rows: rows [0, rows) of
    ``host``, or with ``order`` (int64 host indices) the rows host[order[0]], host[order[1]], ..., gathered into the
    staging buffers as each chunk is read (the solver's shuffled order without a shuffled host copy)."""

    def __init__(self, host: torch.Tensor, device, chunk_rows: int | None = None, order: torch.Tensor | None = None):
        if host.device.type != "cpu" or host.dtype != torch.float32 or host.ndim != 2 or not host.is_contiguous():
            raise ValueError("streamed rows must be a contiguous fp32 host matrix")
        if order is not None:
            order = order.detach().to("cpu", torch.int64).contiguous()
            if order.ndim != 1:
                raise ValueError("order must be a vector of row indices")
        self.host = host
        self.order = order
        self.device = torch.device(device)
        self.rows = int(host.shape[0]) if order is None else int(order.numel())
        self.d = int(host.shape[1])
        self.chunk = int(chunk_rows) if chunk_rows else max(1, STREAM_CHUNK_BYTES // (4 * max(1, self.d)))
        self._copy = None

    @property
    def shape(self):
        return (self.rows, self.d)

    def __len__(self) -> int:
        return self.rows

    def nbytes(self) -> int:
        return 4 * self.rows * self.d

    def prefix(self, rows: int) -> "HostRows":
        if self.order is None:
            return HostRows(self.host[: int(rows)], self.device, self.chunk)
        return HostRows(self.host, self.device, self.chunk, self.order[: int(rows)])

    def _read(self, s: int, e: int, out: torch.Tensor) -> None:
        """Rows [s, e) into ``out`` (host)."""
        if self.order is None:
            out.copy_(self.host[s:e])
        else:
            torch.index_select(self.host, 0, self.order[s:e], out=out)

    def to_device(self) -> torch.Tensor:
        if self.order is None:
            return self.host.to(self.device)
        out = torch.empty((self.rows, self.d), dtype=torch.float32)
        self._read(0, self.rows, out)
        return out.to(self.device)

    def chunks(self, start: int = 0, stop: int | None = None, rows: int | None = None):
        """Yields (s, e, x): x holds rows [s, e) on the device, valid on the current stream until the next step.
        ``rows`` (at most ``chunk``) reads smaller chunks, with smaller buffers. While the caller works on a chunk, a
        worker thread gathers the next one into its staging buffer and queues its upload, so neither the host gather
        nor the upload waits for the caller's work to be queued (the caller's calls synchronise the device)."""
        stop = self.rows if stop is None else int(stop)
        if stop <= start:
            return
        compute = torch.cuda.current_stream(self.device)
        if self._copy is None:
            self._copy = torch.cuda.Stream(self.device)
        copy = self._copy
        rows = min(self.chunk if rows is None else max(1, min(int(rows), self.chunk)), stop - start)
        staging = [torch.empty((rows, self.d), dtype=torch.float32, pin_memory=True) for _ in range(2)]
        buffers = [torch.empty((rows, self.d), dtype=torch.float32, device=self.device) for _ in range(2)]
        uploaded = [torch.cuda.Event(), torch.cuda.Event()]   # staging slot free again / device slot filled
        released = [torch.cuda.Event(), torch.cuda.Event()]   # the caller's work on the device slot is queued before
        used = [False, False]
        bounds = [(s, min(stop, s + rows)) for s in range(start, stop, rows)]
        copy.wait_stream(compute)   # the device buffers were allocated on the caller's stream

        def prepare(index):
            # chunk `index` into slot index % 2: its staging buffer once the slot's previous upload has finished,
            # then its upload once the caller's work on the slot's previous chunk (recorded before this runs)
            slot = index % 2
            s, e = bounds[index]
            if used[slot]:
                uploaded[slot].synchronize()
            self._read(s, e, staging[slot][: e - s])
            with torch.cuda.device(self.device), torch.cuda.stream(copy):
                if used[slot]:
                    copy.wait_event(released[slot])
                buffers[slot][: e - s].copy_(staging[slot][: e - s], non_blocking=True)
                uploaded[slot].record(copy)

        pool = ThreadPoolExecutor(max_workers=1) if len(bounds) > 1 else None
        pending = None
        try:
            prepare(0)
            for index, (s, e) in enumerate(bounds):
                slot = index % 2
                if index + 1 < len(bounds):
                    pending = pool.submit(prepare, index + 1)
                compute.wait_event(uploaded[slot])
                yield s, e, buffers[slot][: e - s]
                released[slot].record(compute)
                used[slot] = True
                if pending is not None:
                    pending.result()   # the next chunk is gathered and its upload queued
                    pending = None
        finally:
            if pending is not None:
                try:
                    pending.result()
                except Exception:   # the caller's own error is the one to report
                    pass
            if pool is not None:
                pool.shutdown(wait=True)
            # later work on the caller's stream (including reuse of the buffers' memory) follows every upload, and
            # the staging buffers are not released while an upload still reads them
            compute.wait_stream(copy)
            copy.synchronize()


def _cycles(perm: torch.Tensor):
    """The cycles of length >= 2 of a permutation, each listed from its smallest element c0 as c0, perm[c0],
    perm[perm[c0]], ... and concatenated: (seq, first) with first[t] the position in seq where t's cycle starts.
    Pointer jumping on the permutation's device (log2 n rounds): the smallest element of each cycle, then each
    element's distance to it."""
    n = perm.numel()
    dev = perm.device
    idx = torch.arange(n, device=dev)
    rounds = max(1, (n - 1).bit_length())
    lead, p = idx.clone(), perm.clone()
    for _ in range(rounds):
        lead = torch.minimum(lead, lead[p])
        p = p[p]
    # steps forward from each element to its cycle's smallest element (0 there)
    is_lead = lead == idx
    dist = (~is_lead).to(torch.int64)
    succ = torch.where(is_lead, idx, perm)
    for _ in range(rounds):
        dist = dist + dist[succ]
        succ = succ[succ]
    length = 1 + dist[perm[lead]]
    moving = length > 1
    rank = torch.remainder(length - dist, length)
    seq = idx[moving][torch.argsort((lead * n + rank)[moving])]
    pos = torch.arange(seq.numel(), device=dev)
    first = torch.cummax(torch.where(rank[seq] == 0, pos, torch.zeros_like(pos)), 0).values
    return seq, first


def permute_rows_inplace(value: torch.Tensor, perm: torch.Tensor, block: int | None = None) -> torch.Tensor:
    """value[i] = (old value)[perm[i]] for a contiguous matrix, on its own device, with one block of extra rows
    instead of a full copy. The permutation's cycles are laid end to end (``_cycles``) and walked in blocks of
    positions: a block gathers the old rows its positions take (the next element of each position's cycle, or for a
    cycle's last element its first), then writes them. A block only reads positions at or after its own, except a
    wrap to a cycle's first element, which an earlier block may have written when the cycle crosses a block
    boundary: those first rows (at most one cycle per boundary) are saved before any write. The role of the
    reference's in-place reorder of consumed inputs (hierarchy/plan.py:13-38), whose temporary is one row."""
    rows, d = int(value.shape[0]), int(value.shape[1])
    if block is None:
        block = max(1, STREAM_CHUNK_BYTES // (value.element_size() * max(1, d)))
    seq, first = _cycles(perm.to(value.device, torch.int64))
    total = seq.numel()
    if total == 0:
        return value
    pos = torch.arange(total, device=value.device)
    nxt = pos + 1
    wrap = nxt >= total
    wrap[:-1] |= first[1:] == nxt[:-1]                  # the next position starts another cycle
    src = torch.where(wrap, first, nxt)
    # wraps whose cycle starts in an earlier block read a saved copy of that cycle's first row
    saved = wrap & (first // block < pos // block)
    starts = torch.unique(first[saved])
    heads = value.index_select(0, seq[starts]) if starts.numel() else None
    temp = torch.empty((min(block, total), d), dtype=value.dtype, device=value.device)
    for t0 in range(0, total, block):
        t1 = min(total, t0 + block)
        out = temp[: t1 - t0]
        torch.index_select(value, 0, seq[src[t0:t1]], out=out)
        m = saved[t0:t1]
        if heads is not None and bool(m.any()):
            out[m] = heads[torch.searchsorted(starts, first[t0:t1][m])]
        value.index_copy_(0, seq[t0:t1], out)
    return value


def shuffled_rows(value, perm: torch.Tensor) -> torch.Tensor:
    """The rows of ``value`` (host or device, any float dtype) in the order ``perm``, as a new fp32 host matrix,
    gathered in bounded row blocks."""
    rows, d = int(value.shape[0]), int(value.shape[1])
    out = torch.empty((rows, d), dtype=torch.float32)
    if torch.is_tensor(value) and value.is_cuda:
        block = max(1, STREAM_CHUNK_BYTES // (4 * max(1, d)))
        perm_dev = perm.to(value.device)
        for s in range(0, rows, block):
            e = min(rows, s + block)
            out[s:e].copy_(value[perm_dev[s:e]].to(torch.float32))
        return out
    host = value if torch.is_tensor(value) else torch.as_tensor(value)
    torch.index_select(host.to(torch.float32), 0, perm.detach().to("cpu", torch.int64), out=out)
    return out


__all__ = ["HostRows", "STREAM_CHUNK_BYTES", "STREAM_MIN_BYTES", "shuffled_rows"]
