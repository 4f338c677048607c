"""Streams and graphs of the HIP runtime libt0g.so itself uses, through ctypes.

libt0g links libamdhip64.so.7 by soname, so loading that name again returns the same
runtime instance (torch's wheel carries a second copy that its own libraries load
under another name; a stream of that copy means nothing to this one).  Test
infrastructure only."""
import ctypes

import t0g  # noqa: F401  (loads libt0g.so, and with it the runtime, first)

_hip = ctypes.CDLL("libamdhip64.so.7")
_vp = ctypes.c_void_p


def _sig(name, *argtypes):
    f = getattr(_hip, name)
    f.restype = ctypes.c_int
    f.argtypes = list(argtypes)
    return f


_sig("hipStreamCreate", ctypes.POINTER(_vp))
_sig("hipStreamDestroy", _vp)
_sig("hipStreamSynchronize", _vp)
_sig("hipStreamBeginCapture", _vp, ctypes.c_int)
_sig("hipStreamEndCapture", _vp, ctypes.POINTER(_vp))
_sig("hipGraphInstantiate", ctypes.POINTER(_vp), _vp, _vp, ctypes.c_char_p, ctypes.c_size_t)
_sig("hipGraphLaunch", _vp, _vp)
_sig("hipGraphExecDestroy", _vp)
_sig("hipGraphDestroy", _vp)

CAPTURE_THREAD_LOCAL = 1   # hipStreamCaptureModeThreadLocal


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


class Stream:
    """A default-priority stream (hipStreamCreate)."""

    def __init__(self):
        self.handle = _vp()
        _ok(_hip.hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    @property
    def ptr(self):
        return self.handle.value

    def synchronize(self):
        _ok(_hip.hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self):
        if self.handle:
            _ok(_hip.hipStreamDestroy(self.handle), "hipStreamDestroy")
            self.handle = _vp()


class Graph:
    """Capture what fn() enqueues on `stream` into an executable graph."""

    def __init__(self, stream, fn):
        self.graph, self.exec = _vp(), _vp()
        _ok(_hip.hipStreamBeginCapture(stream.handle, CAPTURE_THREAD_LOCAL), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            _ok(_hip.hipStreamEndCapture(stream.handle, ctypes.byref(self.graph)), "hipStreamEndCapture")
        _ok(_hip.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")

    def launch(self, stream):
        _ok(_hip.hipGraphLaunch(self.exec, stream.handle), "hipGraphLaunch")

    def destroy(self):
        if self.exec:
            _hip.hipGraphExecDestroy(self.exec)
        if self.graph:
            _hip.hipGraphDestroy(self.graph)
        self.exec = self.graph = _vp()
