"""Capture one fixed-shape inference forward into a hipGraph and replay it.

`CapturedForward(forward, example, warmup=3)` is the drop-in for the
reference's thin_backend/graph.py:6-51: the same constructor, the same
`replay()`, `__call__(value)`, `close()` and `outputs`, and the same exception
types and messages.

How this one works:

* The graph reads its input from one static device tensor, `input`. It is
  allocated with the example's layout and filled from the example.
* `forward` runs `warmup` times eagerly first. This lets the caching allocator
  hold the blocks the capture will reuse, and lets lazily built state (plans,
  flow libraries) settle outside the capture.
* One more call runs under stream capture (`thin_backend::RuntimeGraph`, see
  runtime.cpp). Whatever it returns becomes `outputs`. Those tensors live in
  graph-owned memory, and every replay overwrites them.
* The graph is launched once before the constructor returns, so `outputs`
  already hold the example's results.
* A call with a new value checks it against the captured input's signature.
  It copies the value into `input` and replays.
* Only the creating thread may replay. A graph is bound to that thread's
  stream, and no concurrent replay is supported.
"""
from contextlib import contextmanager
from threading import get_ident
from typing import NamedTuple

import torch

_NOT_INFERENCE = "CapturedForward requires an inference-only NPU input"
_WRONG_THREAD = "RuntimeGraph must stay on its creating thread/stream"
_MISMATCH = "Graph input shape, dtype, device and layout/strides must match capture"


class _InputSignature(NamedTuple):
    """What a replay input must share with the example the graph was captured on."""
    shape: torch.Size
    stride: tuple
    dtype: torch.dtype
    device: torch.device
    layout: torch.layout

    @classmethod
    def of(cls, t: torch.Tensor) -> "_InputSignature":
        return cls(t.shape, t.stride(), t.dtype, t.device, t.layout)

    def admits(self, t: torch.Tensor) -> bool:
        return not t.requires_grad and _InputSignature.of(t) == self


@contextmanager
def _stream_capture(graph):
    """Record the calling thread's stream into `graph` for the duration of the
    block. The capture is ended even when the block raises, for example on a
    device-to-host copy, which cannot be recorded."""
    graph.begin()
    try:
        yield
    finally:
        graph.end()


class CapturedForward:
    """A forward recorded once and replayed on new inputs of the same signature.

    Replays write into the same output tensors (graph-owned memory), so keep a
    clone of any result needed after the next call. The forward, its
    parameters and anything the capture read must stay as they were. Use the
    object from the thread that built it, one replay at a time.
    """

    def __init__(self, forward, example, warmup=3):
        if example.device.type != "npu" or example.requires_grad:
            raise ValueError(_NOT_INFERENCE)
        self._owner = get_ident()
        self._signature = _InputSignature.of(example)
        self.forward = forward
        self.input = torch.empty_like(example)
        self.input.copy_(example)
        self.outputs = None
        self.graph = torch.classes.thin_backend.RuntimeGraph()
        with torch.inference_mode():
            for _ in range(warmup):
                forward(self.input)
            with _stream_capture(self.graph):
                self.outputs = forward(self.input)
        self._launch()

    # -- hooks shared with FrozenGraph
    def _before_launch(self):
        """Called before every replay; FrozenGraph validates its pilot here."""

    def _launch(self):
        self.graph.replay()
        return self.outputs

    # -- public contract
    def replay(self):
        """Launch the graph on whatever `input` holds now; returns `outputs`,
        which the launch overwrites (asynchronously, on this thread's stream)."""
        self._before_launch()
        return self._launch()

    def __call__(self, value):
        self._before_launch()
        if get_ident() != self._owner:
            raise RuntimeError(_WRONG_THREAD)
        if not self._signature.admits(value):
            raise ValueError(_MISMATCH)
        self.input.copy_(value)
        return self._launch()

    def close(self):
        """Release the graph (idempotent). Outputs stay valid as tensors."""
        self.graph.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False
