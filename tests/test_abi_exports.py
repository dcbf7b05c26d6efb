"""CPU checks of the C ABI: the library loads without a GPU, exports every
function include/dcengine.h declares, keeps the reference's struct layouts,
and fails cleanly (no crash, an error string) when no device is initialised."""
import ctypes
import os
import re

import pytest

from directcompute_torch_amd import LIB_PATH, _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "dcengine.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b([A-Z]\w+)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("GPUInfo", "SeqCmd")))


def test_header_declares_reference_exports():
    names = set(declared_functions())
    # the 32 engine.dll exports bound by nn_engine.py:42-121 (+ GetGPUInfo)
    ref = {"InitEngine", "GetGPUInfo", "CreateBuffer", "AddRefBuffer", "ReleaseBuffer",
           "ReleaseBufferBatch", "UpdateBuffer", "ReadBuffer", "ClearBuffer", "FlushGPU", "SyncGPU",
           "WarmPool", "GetPoolStats", "ResetPoolStats", "GetPoolMemory", "DrainPool",
           "CompileShader", "CompileShaderEx", "RunShader", "RunShaderRaw", "RunShaderAlloc",
           "RunShaderAlloc2", "ResolveShader", "RunSequence", "RunSequenceWithSGD", "MatMulAlloc",
           "ConvForwardFused", "ConvBackwardFused", "MaxPoolForwardFused", "MaxPoolBackwardFused",
           "SGDBatch", "SGDBatchClipped"}
    assert ref <= names, sorted(ref - names)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_struct_layouts_match_reference():
    assert ctypes.sizeof(_lib.GPUInfo) == 160
    assert _lib.GPUInfo.description.offset == 28
    assert ctypes.sizeof(_lib.SeqCmd) == 200
    offs = {f: getattr(_lib.SeqCmd, f).offset for f in
            ("shader", "srvs", "srvCount", "uavs", "uavCount", "threads", "cbData", "cbSize")}
    assert offs == {"shader": 0, "srvs": 8, "srvCount": 72, "uavs": 80, "uavCount": 112,
                    "threads": 116, "cbData": 128, "cbSize": 192}


def test_calls_without_init_fail_cleanly():
    """Entry points called before InitEngine return NULL/0 and set an error;
    nothing touches a device (this container has none)."""
    lib = _lib.open_library()
    info = _lib.GPUInfo()
    lib.GetGPUInfo(ctypes.byref(info))
    if info.vendorId != 0:
        pytest.skip("engine already initialised in this process")
    assert lib.CreateBuffer(None, 16) is None
    assert "not initialised" in _lib.last_error(lib)
    assert lib.MatMulAlloc(None, None, 1, 1, 1, 0) is None
    lib.ReleaseBuffer(None)          # NULL is a no-op, as in the reference
    lib.ReleaseBufferBatch(None, 0)
    assert lib.GetPoolMemory() == 0
    assert lib.CompileShader(b"conv_reshape", None)
    assert lib.CompileShader(b"batchnorm_backward_dx", None)
    for name in (b"conv_forward_tiled", b"conv_backprop_filters_tiled", b"conv_backprop_input_fused"):
        assert lib.CompileShader(name, None), name          # nn_engine.py:148
    assert not lib.CompileShader(b"gelu", None)       # no kernel source in the reference
    assert not lib.CompileShaderEx(b"custom", None, b"CSMain")
    assert lib.ResolveShader(b"relu_grad")
    assert lib.ResolveShader(b"no_such_kernel") is None
