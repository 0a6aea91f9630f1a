"""A training step's device work recorded once into a HIP graph and replayed.

A small model's step is a handful of kernels of a few microseconds each.  Issued one by
one from Python, each costs more on the host than it runs on the device: the drop-in
tail of the reference's 1,857-parameter MLP (local share, clip, AdamW; three launches
per rank) spends several times longer in host code than its kernels run.
:class:`StepGraph` records every launch a step function makes into one HIP graph
(``torch.cuda.graph``) and replays them all with one launch.

A replay changes what the eager step would change and nothing else.  The optimizer
kernels of a recorded step read their scalars from small device slots
(``hbt_*_step_slot``), since AdamW's bias corrections move every step and every
scalar follows the learning rate.  Before each replay, :meth:`StepGraph.replay`
formats every recorded step's scalars from the host state (``hbt_*_scalar_record``,
formed as the eager step forms them), writes the slots with one launch per eight of
them (``hbt_write_words``) and advances the step counters, so a replay is bitwise the eager
step.  Copy tables that recorded launches read are written by the
graph itself (``hbt_write_words``) and live as long as it does.

Rules, checked where they can be:

* The step function has run eagerly at least once before it is recorded: the first
  step creates the optimizer state and SGD's momentum buffers.
* It only launches device work.  Parameters or optimizer state in host memory, a
  pending loss-scale factor (the scaler decides on the host whether to skip) and any
  host synchronisation raise while recording.
* Replays read and write the tensors the recording saw.  Write new inputs into them
  (``grad.copy_(...)``) rather than rebinding ``.grad`` (a replay checks the optimizer's
  gradients); tensors the step function allocated and returned (:attr:`StepGraph.output`)
  are refreshed in place by every replay.
* A recording belongs to one device and to torch's current stream at replay time;
  replays of one graph run in order on that stream.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

import torch

from . import _native
from .errors import UnsupportedFeatureError, format_error

__all__ = ["StepGraph"]


class StepGraph:
    """``step()``'s launches recorded into one HIP graph; :meth:`replay` runs them again.

    Recording does not run the step: the graph's first replay is the step after the
    last eager one.  ``pool`` is passed to ``torch.cuda.graph`` (memory-pool sharing
    between graphs).
    """

    def __init__(self, step: Callable[[], Any], *, device: torch.device | None = None, pool: Any = None) -> None:
        if not torch.cuda.is_available():
            raise UnsupportedFeatureError(
                format_error("graphs.StepGraph", "recording a HIP graph needs a HIP device",
                             observed="torch.cuda.is_available() is False")
            )
        self._device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        if self._device.type != "cuda":
            raise UnsupportedFeatureError(
                format_error("graphs.StepGraph", "a HIP graph records device work", observed=str(self._device))
            )
        self._graph = torch.cuda.CUDAGraph()
        recording = _native.GraphRecording(self._device)
        token = _native.set_graph_recording(recording)
        try:
            with torch.cuda.device(self._device), torch.cuda.graph(self._graph, pool=pool):
                self.output = step()
        finally:
            _native.reset_graph_recording(token)
        seen: set[int] = set()
        for recorded in recording.steps:
            for p in recorded.parameters:
                if id(p) in seen:
                    raise UnsupportedFeatureError(
                        format_error("graphs.StepGraph",
                                     "the step function steps a parameter twice; a replay advances each "
                                     "recorded launch by one step from the same host state",
                                     resolution="record a function that steps each optimizer once")
                    )
                seen.add(id(p))
        self._steps = recording.steps
        self._recording = recording  # the slots and device tables the recorded launches read

    @property
    def recorded_steps(self) -> int:
        """Optimizer launch groups whose scalars each replay rewrites."""
        return len(self._steps)

    def replay(self) -> None:
        """Advance every recorded optimizer by one step and run the recorded launches,
        on torch's current stream.  Every recorded step is checked before any is
        advanced, so a refused replay changes nothing."""
        with _native.device_guard(self._device):
            commits = [recorded.prepare() for recorded in self._steps]
            self._recording.write_slots()  # every step's new scalars, in one launch per 8 slots
            for commit in commits:
                commit()
            self._graph.replay()

    def pool(self) -> Any:
        """The graph's memory pool, to share with another recording."""
        return self._graph.pool()
