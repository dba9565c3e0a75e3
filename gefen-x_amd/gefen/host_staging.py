"""Host-resident parameters stepped on the HIP device (CPU offload).

A CPU-offload trainer keeps some parameters, their gradients and their
optimizer state in host memory and pages them between steps.  The reference
steps such a parameter on the host with its decomposed torch-op step and
keeps the state on the parameter's device (gefen.py:66-77, 1897-1927,
tests/test_cpu_resident_step.py).  Here the arithmetic stays on the GPU: the
host parameters of one step are packed into pinned host memory, copied to the
device in one DMA per chunk, stepped by one multi-tensor launch per chunk (the
same kernels, descriptors and rounding as a device-resident parameter), and
the parameter and its state are copied back in one DMA per chunk and written
into the host tensors in place.  The state therefore stays in host memory
between steps, with the parameter, and the results are bit-identical to the
same step of a device-resident parameter.

Layout of one chunk in its arena (pinned host and device alike, every piece
256-byte aligned): first the pieces the step writes (parameter, m_codebook,
m_magnitude, then v_row and v_col, or vmean), then the gradients, which are
only read; the copy back covers the written region alone.  Two arenas
alternate, so the host packs chunk k+1 and unpacks chunk k-1 while the device
works on chunk k.  Chunks hold about GEFENX_HOST_STAGING_BYTES bytes (default
512 MiB); a parameter larger than that takes a chunk of its own.
"""
from __future__ import annotations

import os
from typing import List, Sequence, Tuple

import torch

_ALIGN = 256
DEFAULT_CHUNK_BYTES = 512 << 20


def _round_up(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def chunk_bytes_from_env() -> int:
    raw = os.environ.get("GEFENX_HOST_STAGING_BYTES")
    if raw is None:
        return DEFAULT_CHUNK_BYTES
    value = int(raw)
    if value <= 0:
        raise ValueError("GEFENX_HOST_STAGING_BYTES must be positive, got {}".format(raw))
    return value


class StagedItem:
    """One host parameter of a step: its tensors and where they sit in the
    chunk's arena.  `pieces` lists (key, host tensor, offset) for the written
    region (key "p" is the parameter, the rest are state keys); the gradient
    sits at `grad_offset`."""

    __slots__ = ("group", "name", "p", "grad", "factored", "prepared", "pieces", "grad_offset")

    def __init__(self, group, name, p, grad, factored, prepared):
        self.group, self.name, self.p, self.grad = group, name, p, grad
        self.factored, self.prepared = factored, prepared
        self.pieces: List[Tuple[str, torch.Tensor, int]] = []
        self.grad_offset = 0

    def state_keys(self) -> Tuple[str, ...]:
        base = ("m_codebook", "m_magnitude")
        return base + (("v_row", "v_col") if self.factored else ("vmean",))

    def nbytes(self) -> int:
        state = self.prepared[0]
        sizes = [self.p.numel() * self.p.element_size(), self.grad.numel() * self.grad.element_size()]
        sizes += [state[k].numel() * state[k].element_size() for k in self.state_keys()]
        return sum(_round_up(s) for s in sizes)


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _slice(buf: torch.Tensor, offset: int, like: torch.Tensor) -> torch.Tensor:
    """The arena bytes at `offset` viewed as a contiguous tensor of like's
    dtype and shape."""
    return buf[offset:offset + _nbytes(like)].view(like.dtype).view(like.shape)


class _Chunk:
    def __init__(self, items: Sequence[StagedItem]):
        self.items = list(items)
        off = 0
        for it in self.items:
            state = it.prepared[0]
            it.pieces = []
            for key, t in [("p", it.p)] + [(k, state[k]) for k in it.state_keys()]:
                it.pieces.append((key, t, off))
                off += _round_up(_nbytes(t))
        self.written = off
        for it in self.items:
            it.grad_offset = off
            off += _round_up(_nbytes(it.grad))
        self.total = max(off, _ALIGN)


class HostStager:
    """Pinned and device arenas reused across steps (two of each)."""

    def __init__(self):
        self._pinned = [None, None]
        self._device = {}  # device -> [arena, arena]

    def _pinned_arena(self, slot: int, nbytes: int) -> torch.Tensor:
        buf = self._pinned[slot]
        if buf is None or buf.numel() < nbytes:
            buf = None
            self._pinned[slot] = None
            buf = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
            self._pinned[slot] = buf
        return buf

    def _device_arena(self, device: torch.device, slot: int, nbytes: int) -> torch.Tensor:
        pair = self._device.setdefault(device, [None, None])
        buf = pair[slot]
        if buf is None or buf.numel() < nbytes:
            pair[slot] = None
            buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
            pair[slot] = buf
        return buf

    @staticmethod
    def chunks(items: Sequence[StagedItem], limit: int) -> List[_Chunk]:
        out, cur, size = [], [], 0
        for it in items:
            n = it.nbytes()
            if cur and size + n > limit:
                out.append(_Chunk(cur))
                cur, size = [], 0
            cur.append(it)
            size += n
        if cur:
            out.append(_Chunk(cur))
        return out

    def run(self, items: Sequence[StagedItem], device: torch.device, launch, limit: int) -> None:
        """Step `items` on `device`.  launch(chunk_items, arena) enqueues the
        multi-tensor step of one chunk whose tensors sit in `arena` (a device
        uint8 tensor laid out as the chunk's pieces).  Returns once every
        parameter and state tensor of every item holds its new value."""
        stream = torch.cuda.current_stream(device)
        pending = None
        for k, chunk in enumerate(self.chunks(items, limit)):
            slot = k % 2
            pinned = self._pinned_arena(slot, chunk.total)
            arena = self._device_arena(device, slot, chunk.total)
            # pack: every host tensor into its pinned slot (logical row-major
            # order, so strided host views arrive contiguous)
            for it in chunk.items:
                for _, t, off in it.pieces:
                    _slice(pinned, off, t).copy_(t)
                _slice(pinned, it.grad_offset, it.grad).copy_(it.grad)
            with torch.cuda.device(device):
                arena[:chunk.total].copy_(pinned[:chunk.total], non_blocking=True)
                launch(chunk.items, arena)
                pinned[:chunk.written].copy_(arena[:chunk.written], non_blocking=True)
                done = torch.cuda.Event()
                done.record(stream)
            if pending is not None:
                self._unpack(*pending)
            pending = (chunk, pinned, done)
        if pending is not None:
            self._unpack(*pending)

    @staticmethod
    def _unpack(chunk: _Chunk, pinned: torch.Tensor, done) -> None:
        done.synchronize()
        for it in chunk.items:
            for _, t, off in it.pieces:
                t.copy_(_slice(pinned, off, t))
