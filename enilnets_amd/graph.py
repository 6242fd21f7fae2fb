"""Captured HIP graphs of library calls (``enq_graph_*``).

A serving loop that repeats one fixed sequence of calls (a layer on buffers
it keeps) records it once with ``capture`` and replays it with
``Graph.replay``: one launch instead of one host dispatch per kernel.  No
counterpart in the reference, which runs NumPy on the host."""

import ctypes
from typing import Callable

from . import _lib


class Graph:
    """A captured sequence of library calls."""

    __slots__ = ("_handle",)

    def __init__(self, handle: int):
        self._handle = handle

    def replay(self) -> None:
        """Run the recorded calls again on the library stream."""
        if not self._handle:
            raise ValueError("graph is closed")
        _lib.call("enq_graph_launch", ctypes.c_void_p(self._handle))

    def close(self) -> None:
        """Wait for the stream and free the graph (the library's workspace
        may grow again once no graph is alive)."""
        if self._handle:
            handle, self._handle = self._handle, 0
            _lib.call("enq_graph_destroy", ctypes.c_void_p(handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def capture(fn: Callable[[], None]) -> Graph:
    """Record the library calls ``fn`` makes into a ``Graph`` (they do not run
    now).  Run ``fn`` once before capturing it: while a graph is alive the
    library's workspace does not grow, and the buffers ``fn`` uses must stay
    allocated for as long as the graph is replayed."""
    _lib.call("enq_graph_begin")
    try:
        fn()
    except BaseException:
        handle = ctypes.c_void_p()
        try:
            _lib.call("enq_graph_end", ctypes.byref(handle))
        except Exception:
            pass
        if handle.value:
            _lib.call("enq_graph_destroy", handle)
        raise
    handle = ctypes.c_void_p()
    _lib.call("enq_graph_end", ctypes.byref(handle))
    return Graph(handle.value)
