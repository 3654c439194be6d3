"""Minimal ctypes binding of the HIP runtime calls used for timing and graph
replay (streams, events, stream capture).  Plumbing for bench.py and tests."""
from __future__ import annotations

import ctypes as C

_vp = C.c_void_p


class HipError(RuntimeError):
    pass


class HipRuntime:
    CAPTURE_RELAXED = 2  # hipStreamCaptureModeRelaxed

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        self.L.hipGetErrorString.restype = C.c_char_p

    def _chk(self, rc: int, what: str) -> None:
        if rc != 0:
            raise HipError(f"{what}: {self.L.hipGetErrorString(rc).decode()} ({rc})")

    def stream_create(self) -> int:
        s = _vp()
        self._chk(self.L.hipStreamCreateWithFlags(C.byref(s), C.c_uint(1)), "hipStreamCreateWithFlags")
        return s.value

    def stream_destroy(self, s: int) -> None:
        self._chk(self.L.hipStreamDestroy(_vp(s)), "hipStreamDestroy")

    def stream_sync(self, s: int) -> None:
        self._chk(self.L.hipStreamSynchronize(_vp(s)), "hipStreamSynchronize")

    def event_create(self) -> int:
        e = _vp()
        self._chk(self.L.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def event_record(self, e: int, s: int) -> None:
        self._chk(self.L.hipEventRecord(_vp(e), _vp(s)), "hipEventRecord")

    def event_sync(self, e: int) -> None:
        self._chk(self.L.hipEventSynchronize(_vp(e)), "hipEventSynchronize")

    def elapsed_ms(self, e0: int, e1: int) -> float:
        ms = C.c_float()
        self._chk(self.L.hipEventElapsedTime(C.byref(ms), _vp(e0), _vp(e1)), "hipEventElapsedTime")
        return ms.value

    def capture(self, s: int, fn) -> int:
        """Record everything `fn()` enqueues on stream `s` into an executable graph."""
        self._chk(self.L.hipStreamBeginCapture(_vp(s), C.c_int(self.CAPTURE_RELAXED)), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = _vp()
            rc = self.L.hipStreamEndCapture(_vp(s), C.byref(g))
        self._chk(rc, "hipStreamEndCapture")
        ge = _vp()
        self._chk(self.L.hipGraphInstantiate(C.byref(ge), g, None, None, C.c_size_t(0)), "hipGraphInstantiate")
        self._chk(self.L.hipGraphDestroy(g), "hipGraphDestroy")
        return ge.value

    def graph_upload(self, ge: int, s: int) -> None:
        """hipGraphUpload: the executable graph's one-time device set-up, done
        ahead of its first launch (which otherwise pays for it)."""
        self._chk(self.L.hipGraphUpload(_vp(ge), _vp(s)), "hipGraphUpload")

    def graph_launch(self, ge: int, s: int) -> None:
        self._chk(self.L.hipGraphLaunch(_vp(ge), _vp(s)), "hipGraphLaunch")

    def graph_destroy(self, ge: int) -> None:
        self._chk(self.L.hipGraphExecDestroy(_vp(ge)), "hipGraphExecDestroy")
