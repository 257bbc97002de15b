"""CPU offload of int8 frozen weights (cpu_offload = true, src/layers/quantization.jl:46-64,
111-144; docs/src/training/low_vram.md:46-52).

The reference keeps the QuantizedMatrix codes and scales in host memory. Each forward and
backward call copies them to the GPU (_array_on_input_device: CuArray(Array(values)),
synchronously) and dequantizes them there. Here:

- `offload_weight` keeps a QuantizedMatrix in pinned host memory (page-locked, allocated as
  such), so uploads are asynchronous DMA;
- `upload` (used by i8lora_forward / i8lora_backward for an offloaded weight) is the
  reference's per-call copy, enqueued on the caller's stream;
- `WeightStreamer` overlaps the uploads with compute: device slots hold the codes and scales of
  recently used weights. `prefetch(w)` starts the next weight's upload on a copy stream while
  the current projection computes, and `acquire(w)` makes the compute stream wait for that
  upload only. A slot is overwritten only after the compute stream has finished with it
  (`release` records an event there that the copy stream waits for).

The codes are the same bytes either way, so every output is bit-identical to the resident path.
"""
from __future__ import annotations

from typing import Iterable, List, Optional

import torch

from .layers import QuantizedMatrix


def is_offloaded(w: QuantizedMatrix) -> bool:
    return not w.values.is_cuda


def offload_weight(w: QuantizedMatrix) -> QuantizedMatrix:
    """A copy of w whose codes and scales live in pinned host memory (the reference's host-side
    QuantizedMatrix under cpu_offload, quantization.jl:117-119, 139-140)."""
    v = torch.empty(tuple(w.values.shape), dtype=torch.int8, pin_memory=True)
    s = torch.empty(tuple(w.scales.shape), dtype=torch.float32, pin_memory=True)
    v.copy_(w.values)
    s.copy_(w.scales)
    return QuantizedMatrix(v, s, w.compute_dtype)


def upload(w: QuantizedMatrix, device, stream: Optional[torch.cuda.Stream] = None) -> QuantizedMatrix:
    """_array_on_input_device for an offloaded weight (quantization.jl:46-59): copy codes and
    scales to `device`, enqueued on `stream` (default: the current stream). The returned device
    tensors are ordinary caching-allocator memory that torch keeps alive until the stream's
    work that uses them completes."""
    if not is_offloaded(w):
        return w
    st = stream or torch.cuda.current_stream(device)
    with torch.cuda.stream(st):
        v = torch.empty(tuple(w.values.shape), dtype=torch.int8, device=device)
        s = torch.empty(tuple(w.scales.shape), dtype=torch.float32, device=device)
        v.copy_(w.values, non_blocking=True)
        s.copy_(w.scales, non_blocking=True)
    return QuantizedMatrix(v, s, w.compute_dtype)


class _Slot:
    __slots__ = ("values", "scales", "owner", "ready", "free", "busy")

    def __init__(self):
        self.values = self.scales = None
        self.owner = None  # the host weight held (by identity; kept alive while held)
        self.ready = self.free = None
        self.busy = False


class WeightStreamer:
    """Double-buffered (or deeper, `slots`) uploads of offloaded weights, overlapped with compute.

    Use per projection, in compute order:
        streamer.prefetch(next_weight)   # starts its upload on the copy stream
        W = streamer.acquire(weight)     # device QuantizedMatrix; compute stream waits for it
        ... launch the projection's kernels on the current stream with W ...
        streamer.release(weight)         # the slot may be overwritten after this work

    A weight still held in a slot is not uploaded again (the backward pass starts with the
    forward pass's last projection). Slot buffers grow to the largest weight seen; they are
    allocated once and reused. The copy stream has the default priority."""

    def __init__(self, device, slots: int = 2):
        if slots < 2:
            raise ValueError("WeightStreamer needs at least two slots to overlap uploads")
        self.device = torch.device(device)
        self.copy_stream = torch.cuda.Stream(self.device)
        self.slots: List[_Slot] = [_Slot() for _ in range(slots)]
        self._lru: List[int] = list(range(slots))  # least recently used first
        self.uploads = 0

    def _find(self, w: QuantizedMatrix) -> Optional[int]:
        for i, sl in enumerate(self.slots):
            if sl.owner is w:
                return i
        return None

    def _touch(self, i: int) -> None:
        self._lru.remove(i)
        self._lru.append(i)

    def prefetch(self, w: QuantizedMatrix) -> None:
        """Start uploading w into a free slot, unless it is resident already or on the device."""
        if not is_offloaded(w) or self._find(w) is not None:
            return
        idx = next((i for i in self._lru if not self.slots[i].busy), None)
        if idx is None:
            raise RuntimeError("every WeightStreamer slot is held: release a weight first")
        sl = self.slots[idx]
        nv, ns = w.values.numel(), w.scales.numel()
        with torch.cuda.stream(self.copy_stream):
            if sl.free is not None:
                self.copy_stream.wait_event(sl.free)  # its last reader has finished
            if sl.values is None or sl.values.numel() < nv:
                sl.values = torch.empty((nv,), dtype=torch.int8, device=self.device)
            if sl.scales is None or sl.scales.numel() < ns:
                sl.scales = torch.empty((ns,), dtype=torch.float32, device=self.device)
            sl.values[:nv].copy_(w.values.reshape(-1), non_blocking=True)
            sl.scales[:ns].copy_(w.scales, non_blocking=True)
            sl.ready = torch.cuda.Event()
            sl.ready.record(self.copy_stream)
        sl.owner = w
        sl.free = None
        self.uploads += 1
        self._touch(idx)

    def acquire(self, w: QuantizedMatrix) -> QuantizedMatrix:
        """The device copy of w; the current stream waits for its upload."""
        if not is_offloaded(w):
            return w
        idx = self._find(w)
        if idx is None:
            self.prefetch(w)
            idx = self._find(w)
        sl = self.slots[idx]
        sl.busy = True
        self._touch(idx)
        cur = torch.cuda.current_stream(self.device)
        cur.wait_event(sl.ready)
        sl.values.record_stream(cur)  # the allocator must not recycle these under the compute
        sl.scales.record_stream(cur)
        N, K = w.values.shape
        return QuantizedMatrix(sl.values[: N * K].view(N, K), sl.scales[:N], w.compute_dtype)

    def release(self, w: QuantizedMatrix) -> None:
        """Work enqueued so far on the current stream is the last use of w's slot for now."""
        idx = self._find(w)
        if idx is None:
            return
        sl = self.slots[idx]
        sl.free = torch.cuda.Event()
        sl.free.record(torch.cuda.current_stream(self.device))
        sl.busy = False


class PerCallUploader:
    """The reference's behaviour (no overlap): every acquire copies the weight on the compute
    stream right before its use (_array_on_input_device per call). Same interface as
    WeightStreamer, for comparisons."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.uploads = 0

    def prefetch(self, w: QuantizedMatrix) -> None:
        pass

    def acquire(self, w: QuantizedMatrix) -> QuantizedMatrix:
        if is_offloaded(w):
            self.uploads += 1
        return upload(w, self.device)

    def release(self, w: QuantizedMatrix) -> None:
        pass


def run_streamed(weights: Iterable[QuantizedMatrix], fn, streamer: WeightStreamer) -> list:
    """Calls fn(i, device_weight) for each weight in order, uploading weight i+1 while weight i
    computes. Returns fn's results."""
    ws = list(weights)
    out = []
    if ws:
        streamer.prefetch(ws[0])
    for i, w in enumerate(ws):
        dw = streamer.acquire(w)
        if i + 1 < len(ws):
            streamer.prefetch(ws[i + 1])
        out.append(fn(i, dw))
        streamer.release(w)
    return out
