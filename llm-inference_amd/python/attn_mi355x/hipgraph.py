"""Minimal HIP graph capture/replay through ctypes (tests and bench), for exercising the
update_*_node entry points the way model_inference.hpp:96-126 does.  Binds the
HIP runtime already loaded by torch (same SONAME, one runtime per process)."""
from __future__ import annotations

import ctypes

import torch  # noqa: F401  (loads the HIP runtime first)

_hip = ctypes.CDLL("libamdhip64.so.7")
_vp = ctypes.c_void_p

_hip.hipStreamBeginCapture.argtypes = [_vp, ctypes.c_int]
_hip.hipStreamEndCapture.argtypes = [_vp, ctypes.POINTER(_vp)]
_hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(_vp), _vp, _vp, _vp, ctypes.c_size_t]
_hip.hipGraphLaunch.argtypes = [_vp, _vp]
_hip.hipGraphExecDestroy.argtypes = [_vp]
_hip.hipGraphDestroy.argtypes = [_vp]
_hip.hipStreamSynchronize.argtypes = [_vp]
_hip.hipStreamGetCaptureInfo_v2.argtypes = [_vp, ctypes.POINTER(ctypes.c_int), _vp, _vp,
                                            ctypes.POINTER(ctypes.POINTER(_vp)),
                                            ctypes.POINTER(ctypes.c_size_t)]

CAPTURE_MODE_RELAXED = 2


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed: hipError {rc}")


def begin_capture(stream: int):
    check(_hip.hipStreamBeginCapture(stream, CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")


def last_captured_node(stream: int) -> int:
    """gpu_utils.hpp:45-59: the single current capture dependency."""
    status = ctypes.c_int(0)
    deps = ctypes.POINTER(_vp)()
    count = ctypes.c_size_t(0)
    check(_hip.hipStreamGetCaptureInfo_v2(stream, ctypes.byref(status), None, None,
                                          ctypes.byref(deps), ctypes.byref(count)),
          "hipStreamGetCaptureInfo_v2")
    if status.value != 1 or count.value != 1:
        raise RuntimeError("Expected one capture dependency")
    return deps[0]


def end_capture(stream: int):
    graph = _vp()
    check(_hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
    exe = _vp()
    check(_hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
    return graph, exe


def launch(exe, stream: int):
    check(_hip.hipGraphLaunch(exe, stream), "hipGraphLaunch")


def synchronize(stream: int):
    check(_hip.hipStreamSynchronize(stream), "hipStreamSynchronize")


def destroy(graph, exe):
    _hip.hipGraphExecDestroy(exe)
    _hip.hipGraphDestroy(graph)
