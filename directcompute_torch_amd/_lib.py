"""ctypes binding of libdcengine.so.

The argtypes/restype blocks mirror the reference's binding of engine.dll
(nn_engine.py:42-121) symbol for symbol, plus the additions declared in
include/dcengine.h (GetLastErrorString, AdamBatch, ClipGradNorm, profiling).

Loading never falls back to anything: if the library is missing or no HIP
device is usable, :func:`load` raises.
"""
from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libdcengine.so")

c_void_p = ctypes.c_void_p
c_uint = ctypes.c_uint
c_float = ctypes.c_float
P = ctypes.POINTER


class GPUInfo(ctypes.Structure):
    """engine.cpp GPUInfo layout (160 bytes)."""
    _fields_ = [
        ("vendorId", ctypes.c_uint),
        ("deviceId", ctypes.c_uint),
        ("dedicatedVRAM", ctypes.c_uint64),
        ("sharedMemory", ctypes.c_uint64),
        ("isIntegrated", ctypes.c_uint),
        ("description", ctypes.c_char * 128),
    ]


class SeqCmd(ctypes.Structure):
    """engine.cpp SeqCmd layout (200 bytes)."""
    _fields_ = [
        ("shader", c_void_p),
        ("srvs", c_void_p * 8),
        ("srvCount", c_uint),
        ("uavs", c_void_p * 4),
        ("uavCount", c_uint),
        ("threads", c_uint * 3),
        ("cbData", ctypes.c_uint8 * 64),
        ("cbSize", c_uint),
        ("pad", c_uint * 1),
    ]


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    """Set argtypes/restypes on a loaded library (no device calls)."""
    lib.InitEngine.argtypes = []
    lib.InitEngine.restype = ctypes.c_bool
    lib.GetGPUInfo.argtypes = [P(GPUInfo)]
    lib.GetGPUInfo.restype = None
    lib.CompileShader.argtypes = [ctypes.c_char_p, ctypes.c_wchar_p]
    lib.CompileShader.restype = ctypes.c_bool
    lib.CompileShaderEx.argtypes = [ctypes.c_char_p, ctypes.c_wchar_p, ctypes.c_char_p]
    lib.CompileShaderEx.restype = ctypes.c_bool
    lib.CreateBuffer.argtypes = [P(c_float), c_uint]
    lib.CreateBuffer.restype = c_void_p
    lib.AddRefBuffer.argtypes = [c_void_p]
    lib.AddRefBuffer.restype = None
    lib.ReadBuffer.argtypes = [c_void_p, P(c_float)]
    lib.ReadBuffer.restype = None
    lib.ReleaseBuffer.argtypes = [c_void_p]
    lib.ReleaseBuffer.restype = None
    lib.ClearBuffer.argtypes = [c_void_p]
    lib.ClearBuffer.restype = None
    lib.UpdateBuffer.argtypes = [c_void_p, P(c_float)]
    lib.UpdateBuffer.restype = None
    shader_args = [ctypes.c_char_p, P(c_void_p), c_uint, P(c_void_p), c_uint, P(c_uint), c_void_p, c_uint]
    lib.RunShader.argtypes = shader_args
    lib.RunShader.restype = None
    lib.RunShaderRaw.argtypes = shader_args
    lib.RunShaderRaw.restype = None
    lib.RunShaderAlloc.argtypes = [ctypes.c_char_p, P(c_void_p), c_uint, c_uint, P(c_uint), c_void_p, c_uint]
    lib.RunShaderAlloc.restype = c_void_p
    lib.RunShaderAlloc2.argtypes = [ctypes.c_char_p, P(c_void_p), c_uint, c_uint, c_void_p, P(c_uint), c_void_p, c_uint]
    lib.RunShaderAlloc2.restype = c_void_p
    lib.SGDBatch.argtypes = [P(c_void_p), P(c_void_p), P(c_uint), c_uint, c_float, c_float]
    lib.SGDBatch.restype = None
    lib.SGDBatchClipped.argtypes = [P(c_void_p), P(c_void_p), P(c_uint), c_uint, c_float, c_float]
    lib.SGDBatchClipped.restype = c_float
    lib.ReleaseBufferBatch.argtypes = [P(c_void_p), c_uint]
    lib.ReleaseBufferBatch.restype = None
    lib.FlushGPU.argtypes = []
    lib.FlushGPU.restype = None
    lib.SyncGPU.argtypes = []
    lib.SyncGPU.restype = None
    lib.MatMulAlloc.argtypes = [c_void_p, c_void_p, c_uint, c_uint, c_uint, c_uint]
    lib.MatMulAlloc.restype = c_void_p
    lib.ConvForwardFused.argtypes = [c_void_p, c_void_p, c_void_p] + [c_uint] * 10 + [P(c_void_p)]
    lib.ConvForwardFused.restype = c_void_p
    lib.ConvBackwardFused.argtypes = [c_void_p] * 5 + [c_uint] * 13 + [P(c_void_p)] * 3
    lib.ConvBackwardFused.restype = None
    lib.MaxPoolForwardFused.argtypes = [c_void_p] + [c_uint] * 6 + [P(c_void_p)]
    lib.MaxPoolForwardFused.restype = c_void_p
    lib.MaxPoolBackwardFused.argtypes = [c_void_p, c_void_p] + [c_uint] * 5
    lib.MaxPoolBackwardFused.restype = c_void_p
    lib.WarmPool.argtypes = [P(c_uint), c_uint, c_uint]
    lib.WarmPool.restype = None
    lib.GetPoolStats.argtypes = [P(ctypes.c_uint64), P(ctypes.c_uint64)]
    lib.GetPoolStats.restype = None
    lib.ResetPoolStats.argtypes = []
    lib.ResetPoolStats.restype = None
    lib.GetPoolMemory.argtypes = []
    lib.GetPoolMemory.restype = ctypes.c_uint64
    lib.DrainPool.argtypes = []
    lib.DrainPool.restype = None
    lib.ResolveShader.argtypes = [ctypes.c_char_p]
    lib.ResolveShader.restype = c_void_p
    lib.RunSequence.argtypes = [c_void_p, c_uint]
    lib.RunSequence.restype = None
    lib.RunSequenceWithSGD.argtypes = [c_void_p, c_uint, P(c_void_p), P(c_void_p), P(c_uint), c_uint, c_float, c_float]
    lib.RunSequenceWithSGD.restype = None
    # additions
    lib.GetLastErrorString.argtypes = []
    lib.GetLastErrorString.restype = ctypes.c_char_p
    lib.ClearLastError.argtypes = []
    lib.ClearLastError.restype = None
    lib.AdamBatch.argtypes = [P(c_void_p)] * 4 + [P(c_uint), c_uint] + [c_float] * 6
    lib.AdamBatch.restype = None
    lib.ClipGradNorm.argtypes = [P(c_void_p), P(c_uint), c_uint, c_float]
    lib.ClipGradNorm.restype = c_float
    lib.ClipGradNormNoAlloc.argtypes = [P(c_void_p), P(c_uint), c_uint, c_float]
    lib.ClipGradNormNoAlloc.restype = c_float
    lib.AdamBatchCounted.argtypes = ([P(c_void_p)] * 4 + [P(c_uint), c_uint, c_void_p, c_uint, c_float]
                                     + [ctypes.c_double] * 3 + [c_float] * 3)
    lib.AdamBatchCounted.restype = None
    lib.SetProfiling.argtypes = [ctypes.c_int]
    lib.SetProfiling.restype = None
    lib.GetProfile.argtypes = [ctypes.c_char_p, P(ctypes.c_uint64), P(ctypes.c_double), P(ctypes.c_double), P(ctypes.c_double)]
    lib.GetProfile.restype = ctypes.c_bool
    lib.SetProfileFilter.argtypes = [ctypes.c_char_p]
    lib.SetProfileFilter.restype = None
    lib.BeginCapture.argtypes = []
    lib.BeginCapture.restype = ctypes.c_bool
    lib.EndCapture.argtypes = []
    lib.EndCapture.restype = c_void_p
    lib.ReplayGraph.argtypes = [c_void_p]
    lib.ReplayGraph.restype = ctypes.c_bool
    lib.ReleaseGraph.argtypes = [c_void_p]
    lib.ReleaseGraph.restype = None
    lib.BeginProfileRegion.argtypes = [ctypes.c_char_p, ctypes.c_double, ctypes.c_double]
    lib.BeginProfileRegion.restype = ctypes.c_bool
    lib.EndProfileRegion.argtypes = []
    lib.EndProfileRegion.restype = ctypes.c_bool
    lib.SetStreamingThreshold.argtypes = [ctypes.c_double]
    lib.SetStreamingThreshold.restype = ctypes.c_double
    lib.ResetProfile.argtypes = []
    lib.ResetProfile.restype = None
    return lib


def open_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """dlopen + bind, without touching the GPU."""
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m directcompute_torch_amd.build`")
    return bind(ctypes.CDLL(path))


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Open the library and initialise the engine; raises if no HIP device."""
    lib = open_library(path)
    if not lib.InitEngine():
        raise RuntimeError("libdcengine InitEngine failed: " + lib.GetLastErrorString().decode())
    return lib


def last_error(lib) -> str:
    return lib.GetLastErrorString().decode(errors="replace")
