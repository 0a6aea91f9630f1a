"""Host-resident tensors streamed through device staging buffers.

No kernel of this package reads host memory.  Optimizer state kept on the host
(``cpu_offload_state``), parameter shards kept on the host (``cpu_offload_params``) and
the gradients of those shards reach the kernels through device staging buffers, chunk
by chunk, on two streams of the pass's own: the upload stream copies chunk ``c`` in and
runs its kernel, while the download stream writes chunk ``c - 1`` back, so the two link
directions stay busy at once.  Two staging slots per operand bound the device memory a
pass uses to ``2 * operands * (chunk_elems + lead) * element size``.

The caller's (compute) stream takes no part inside a pass: the pass starts after the
work already queued on it, and work queued on it afterwards waits for the pass's last
write-back, so device-side consumers need no synchronisation.  Host-side readers of
what a pass wrote call :meth:`HostStream.synchronize` first.

The two directions overlap only when the HIP runtime gives the two streams' copies
separate copy resources, and which it gives a stream depends on what other streams of
the process copied before it: measured on MI355X, a pair of streams that was the second
pair to copy in its process ran a 1e9-parameter AdamW pass in 564 ms against 339 ms,
its directions serialised, while the first and third pairs overlapped.  The copies run
as the runtime's blit kernels on the streams' hardware queues (four per process unless
GPU_MAX_HW_QUEUES says otherwise), and two streams on one queue run in order; with 16
queues those pairs overlapped.  Nothing here can choose the queue; one stream pair per
device, created once, keeps the assignment stable for the life of the process.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

__all__ = ["HostOperand", "HostStream", "chunk_plan", "host_stream", "is_host"]


def is_host(tensor: torch.Tensor) -> bool:
    """Whether ``tensor`` lives in host memory."""
    return tensor.device.type == "cpu"


@dataclass(frozen=True)
class HostOperand:
    """One host tensor of a streamed pass: a dense flat view of the pass's elements.

    ``load``: each chunk is uploaded before its launch.  ``store``: each chunk is written
    back after its launch.
    """

    host: torch.Tensor
    load: bool = True
    store: bool = False


def chunk_plan(total: int, chunk: int) -> list[tuple[int, int]]:
    """``(start, n)`` of every chunk of a ``total``-element pass in ``chunk``-element steps."""
    if chunk <= 0:
        raise ValueError(f"chunk must be positive, got {chunk}")
    return [(start, min(chunk, total - start)) for start in range(0, total, chunk)]


class HostStream:
    """Copy streams and staging buffers for passes over host-resident tensors on one device."""

    #: Elements per chunk (128 MB of fp32 per operand and slot).
    chunk_elems = 1 << 25
    slots = 2
    #: Largest ``lead`` a pass may ask for (elements before a staged chunk).
    max_lead = 8

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self.upload = torch.cuda.Stream(self.device)
        self.download = torch.cuda.Stream(self.device)
        self._staging: dict[tuple[int, int], torch.Tensor] = {}
        self.done: torch.cuda.Event | None = None

    def _buffers(self, operands: Sequence[HostOperand], capacity: int) -> list[list[torch.Tensor]]:
        """Byte buffers per slot and operand holding ``capacity`` elements of its dtype.

        Buffers only grow, and only here, before the pass's first copy: a buffer freed
        here was last used by an earlier pass, which the compute stream (the
        allocation's stream) has already waited for.
        """
        out = []
        for slot in range(self.slots):
            row = []
            for k, op in enumerate(operands):
                need = capacity * op.host.element_size()
                buf = self._staging.get((slot, k))
                if buf is None or buf.numel() < need:
                    buf = torch.empty(need, dtype=torch.uint8, device=self.device)
                    self._staging[(slot, k)] = buf
                row.append(buf)
            out.append(row)
        return out

    def run(
        self,
        total: int,
        operands: Sequence[HostOperand],
        launch: Callable[[int, int, list[torch.Tensor], int], None],
        *,
        lead: int = 0,
        chunk: int | None = None,
        resident: tuple[torch.Tensor, torch.Tensor] | None = None,
    ) -> None:
        """Call ``launch(start, n, staged, stream)`` for every chunk ``[start, start + n)``
        of a ``total``-element pass; ``stream`` is the raw ``hipStream_t`` the chunk's
        kernels go on (the upload stream, after the chunk's copies).

        ``staged[k]`` is the device copy of ``operands[k].host[start : start + n]``.  It
        begins ``lead`` elements into its staging buffer, whose base is 256-byte aligned,
        so a kernel that takes a vector path only on 16-byte aligned addresses sees the
        same alignment as on the host tensor when ``lead`` is that tensor's element
        offset from a 16-byte boundary.  ``resident = (device_flat, host_flat)``: after
        each launch, ``device_flat[start : start + n]`` is also written back to
        ``host_flat`` (a device tensor whose host copy follows it).
        """
        if total <= 0:
            return
        chunk = self.chunk_elems if chunk is None else chunk
        if not 0 <= lead < self.max_lead:
            raise ValueError(f"lead must be in [0, {self.max_lead}), got {lead}")
        flats = [op.host.detach().reshape(-1) for op in operands]
        for flat in flats:
            if flat.numel() != total or not is_host(flat):
                raise ValueError("every operand must be a host tensor of the pass's length")
        plan = chunk_plan(total, chunk)
        buffers = self._buffers(operands, lead + plan[0][1])
        compute = torch.cuda.current_stream(self.device)
        free: list[torch.cuda.Event | None] = [None] * self.slots
        self.upload.wait_stream(compute)  # earlier passes and kernels are done
        try:
            self._chunks(plan, operands, flats, buffers, lead, launch, resident, free)
        finally:
            # also after a failed launch: the copies already queued stay ordered before
            # whatever the caller's stream does next
            self.download.wait_stream(self.upload)
            end = torch.cuda.Event()
            end.record(self.download)
            compute.wait_event(end)  # later device work sees the finished copies
            self.done = end

    def _chunks(self, plan, operands, flats, buffers, lead, launch, resident, free) -> None:
        for index, (start, n) in enumerate(plan):
            slot = index % self.slots
            staged = [
                buf[lead * f.element_size() : (lead + n) * f.element_size()].view(f.dtype)
                for buf, f in zip(buffers[slot], flats)
            ]
            computed = torch.cuda.Event()
            with torch.cuda.stream(self.upload):
                if free[slot] is not None:
                    self.upload.wait_event(free[slot])  # the slot's previous chunk is written back
                for op, d, h in zip(operands, staged, flats):
                    if op.load:
                        d.copy_(h[start : start + n], non_blocking=True)
                launch(start, n, staged, self.upload.cuda_stream)
                computed.record(self.upload)
            released = torch.cuda.Event()
            with torch.cuda.stream(self.download):
                self.download.wait_event(computed)
                for op, d, h in zip(operands, staged, flats):
                    if op.store:
                        h[start : start + n].copy_(d, non_blocking=True)
                if resident is not None:
                    device_flat, host_flat = resident
                    host_flat[start : start + n].copy_(device_flat[start : start + n], non_blocking=True)
                released.record(self.download)
            free[slot] = released

    def synchronize(self) -> None:
        """Block the host until the last pass's write-back has landed."""
        if self.done is not None:
            self.done.synchronize()


_STREAMS: dict[int, HostStream] = {}


def release_streams() -> None:
    """Forget every device's :class:`HostStream` (streams, events and staging buffers);
    the next pass creates a new one.  Called at interpreter exit, after the devices have
    been synchronised."""
    _STREAMS.clear()


def host_stream(device: torch.device) -> HostStream:
    """The :class:`HostStream` of ``device`` (one per device, shared by every pass)."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _STREAMS.get(index)
    if stream is None:
        stream = HostStream(torch.device("cuda", index))
        _STREAMS[index] = stream
    return stream
