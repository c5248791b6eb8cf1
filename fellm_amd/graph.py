"""HIP graph capture and replay through the library's C ABI
(``fellm_rocm_graph_*``; replaces crates/backend-cuda/src/graph.rs).

A capture records every launch enqueued on one stream between ``begin`` and
``finish``; the executable replays them with the same kernel arguments.  Per-
step values live in device memory (positions, row lengths, the
DeviceStepParams block), so the host updates that memory between replays.

Launches recorded into a graph must not allocate: pass every output tensor
explicitly (``out=``), since a tensor allocated during the capture can be
freed and reused while the graph still writes to it.  Capture on a
non-default stream (``torch.cuda.Stream()``); the null stream cannot be
captured.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib


class GraphExec:
    """An instantiated graph (CudaGraphExec)."""

    def __init__(self, handle: int):
        self._h = handle

    def launch(self, stream: torch.cuda.Stream | None = None) -> None:
        s = (stream or torch.cuda.current_stream()).cuda_stream
        _lib.call("fellm_rocm_graph_launch", self._h, s)

    def close(self) -> None:
        if self._h:
            _lib.lib().fellm_rocm_graph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GraphCapture:
    """Capture of one stream (CudaGraphCapture).  As a context manager the
    capture is abandoned (stream left out of capture mode) if the body raises."""

    def __init__(self, stream: torch.cuda.Stream):
        self.stream = stream
        self.graph: GraphExec | None = None
        self._active = False

    def begin(self) -> "GraphCapture":
        _lib.call("fellm_rocm_graph_begin", self.stream.cuda_stream)
        self._active = True
        return self

    def finish(self) -> GraphExec:
        h = C.c_void_p()
        self._active = False
        _lib.call("fellm_rocm_graph_end", self.stream.cuda_stream, C.byref(h))
        self.graph = GraphExec(h.value)
        return self.graph

    def abort(self) -> None:
        if self._active:
            self._active = False
            _lib.lib().fellm_rocm_graph_abort(self.stream.cuda_stream)

    def __enter__(self) -> "GraphCapture":
        self._ctx = torch.cuda.stream(self.stream)
        self._ctx.__enter__()
        return self.begin()

    def __exit__(self, exc_type, exc, tb) -> bool:
        try:
            if exc_type is None:
                self.finish()
            else:
                self.abort()
        finally:
            self._ctx.__exit__(exc_type, exc, tb)
        return False


def is_capturing(stream: torch.cuda.Stream) -> bool:
    rc = _lib.lib().fellm_rocm_stream_is_capturing(stream.cuda_stream)
    if rc < 0:
        raise _lib.FellmRocmError("fellm_rocm_stream_is_capturing", rc)
    return rc == 1
