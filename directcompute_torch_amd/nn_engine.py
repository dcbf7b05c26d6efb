"""MI355X backend with the ``nn_engine`` API of raviadi12/directcompute_torch.

Same public surface as the reference module (Tensor / Function autograd,
functional ops, layers, Model, SGD / AdamW / Adam, Metrics, end_batch, pool
helpers), driving ``libdcengine.so`` through ctypes instead of engine.dll.
The buffer-handle protocol is the reference's: every op asks the library for
new handles, ``Tensor.from_gpu`` wraps them, ``_accumulate_grad`` aliases the
first gradient and adds later ones in place (nn_engine.py:575-610).

Importing this module initialises the HIP device (as the reference
initialises D3D11 at import, nn_engine.py:121) and raises if that fails --
there is no CPU fallback.

Not provided (outside the backward path): custom HLSL shaders, the
GELU / LayerNorm / attention family (their kernels do not exist in the
reference tree), ONNX export/import, Muon, and the Python-side profilers.
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np

from . import _lib

lib = _lib.load()
GPUInfo = _lib.GPUInfo


def float_to_uint(f):
    """Bit pattern of a float32 as u32 (nn_engine.py:10-11)."""
    return struct.unpack("I", struct.pack("f", f))[0]


_gpu_info = GPUInfo()
lib.GetGPUInfo(ctypes.byref(_gpu_info))
_IS_IGPU = bool(_gpu_info.isIntegrated)
_GPU_VENDOR = {0x8086: "Intel", 0x10DE: "NVIDIA", 0x1002: "AMD"}.get(
    _gpu_info.vendorId, f"0x{_gpu_info.vendorId:04X}")
_GPU_NAME = _gpu_info.description.decode("ascii", errors="replace").strip("\x00")
_VRAM_MB = _gpu_info.dedicatedVRAM // (1024 * 1024)
_SHARED_MB = _gpu_info.sharedMemory // (1024 * 1024)

# Kernel names the reference compiles at import (nn_engine.py:147-173).  No
# shader source is compiled here; CompileShader only reports whether the
# library implements the name, and (as in the reference) the result is not
# required for names that are never dispatched.
shaders = [
    "matmul_universal", "matmul_coarsened", "matmul_heavy", "add_bias", "relu", "relu_grad",
    "softmax", "softmax_ce_grad", "bias_grad", "sgd", "loss",
    "conv_forward_tiled", "conv_backprop_filters_tiled", "conv_backprop_input_fused", "maxpool_forward",
    "maxpool_backward", "grad_accum", "im2col", "conv_reshape", "conv_grad_reshape", "col2im",
    "argmax_correct", "accumulate_scalar", "bias_relu", "conv_grad_reshape_relu",
    "batchnorm_mean_var", "batchnorm_forward", "batchnorm_backward_reduce",
    "batchnorm_backward_dx", "adam", "scale_add", "rms", "depthwise_conv_forward",
    "depthwise_conv_backward_input", "depthwise_conv_backward_filter", "global_avg_pool",
    "global_avg_pool_backward", "add", "relu6", "relu6_grad", "leaky_relu", "leaky_relu_grad",
    "upsample", "upsample_backward", "concat_insert", "slice", "dice_loss", "dice_loss_grad",
    "sigmoid", "sigmoid_grad", "matmul_reduce", "dice_loss_sums", "grad_sq_reduce",
    "grad_norm_final", "sgd_clipped", "matmul_dgpu",
]
_MISSING_KERNELS = [s for s in shaders if not lib.CompileShader(s.encode(), None)]
if _MISSING_KERNELS:
    raise RuntimeError(f"libdcengine lacks kernels: {_MISSING_KERNELS}")


def last_error():
    """Reason for the library's last failure ('' if none)."""
    return _lib.last_error(lib)


def _check(handle, what):
    if not handle:
        raise RuntimeError(f"{what} failed: {last_error()}")
    return handle


# --------------------------------------------------------------------------
# Dispatch helpers (same packing as nn_engine.py:421-448)
# --------------------------------------------------------------------------
class ParamsCB(ctypes.Structure):
    _fields_ = [(f"u{i}", ctypes.c_uint) for i in range(1, 10)]


_srv_arr = (ctypes.c_void_p * 8)()
_uav_arr = (ctypes.c_void_p * 8)()
_threads = (ctypes.c_uint * 3)()
_cb = ParamsCB()


def _fill(srvs, uavs, tx, ty, tz, vals):
    for i, h in enumerate(srvs):
        _srv_arr[i] = h
    for i, h in enumerate(uavs):
        _uav_arr[i] = h
    _threads[0], _threads[1], _threads[2] = tx, ty, tz
    (_cb.u1, _cb.u2, _cb.u3, _cb.u4, _cb.u5, _cb.u6, _cb.u7, _cb.u8, _cb.u9) = vals


def _dispatch(name, srvs, uavs, tx, ty, tz, u1=0, u2=0, u3=0, u4=0, u5=0, u6=0, u7=0, u8=0, u9=0,
              cbSize=16):
    """RunShader with pre-allocated ctypes arrays."""
    _fill(srvs, uavs, tx, ty, tz, (u1, u2, u3, u4, u5, u6, u7, u8, u9))
    if cbSize > 0:
        lib.RunShader(name, _srv_arr, len(srvs), _uav_arr, len(uavs), _threads, ctypes.byref(_cb), cbSize)
    else:
        lib.RunShader(name, _srv_arr, len(srvs), _uav_arr, len(uavs), _threads, None, 0)


def _dispatch_raw(name, srvs, uavs, tx, ty, tz, u1=0, u2=0, u3=0, u4=0, u5=0, u6=0, u7=0, u8=0,
                  u9=0, cbSize=16):
    """RunShaderRaw with pre-allocated ctypes arrays."""
    _fill(srvs, uavs, tx, ty, tz, (u1, u2, u3, u4, u5, u6, u7, u8, u9))
    if cbSize > 0:
        lib.RunShaderRaw(name, _srv_arr, len(srvs), _uav_arr, len(uavs), _threads, ctypes.byref(_cb), cbSize)
    else:
        lib.RunShaderRaw(name, _srv_arr, len(srvs), _uav_arr, len(uavs), _threads, None, 0)


_all_tensors = []


def release_all_buffers():
    """Detach graph state of every tracked tensor and release their buffers
    with one ReleaseBufferBatch call (nn_engine.py:486-505)."""
    global _all_tensors
    handles = []
    for t in _all_tensors:
        if t._ctx:
            t._ctx.inputs = ()
            t._ctx = None
        t.grad = None
        # A cached traversal order contains the tensor itself: dropping it
        # breaks that cycle, so the tensors it lists (untracked views such as
        # Flatten's, which hold a reference on their buffer) are freed now
        # rather than by a later cyclic garbage collection, and their buffers
        # are back in the pool before the next step asks for them.
        try:
            del t._cached_topo
        except AttributeError:
            pass
        if t.gpu_buf:
            handles.append(t.gpu_buf)
            t.gpu_buf = None
    _all_tensors = []
    if handles:
        arr = (ctypes.c_void_p * len(handles))(*handles)
        lib.ReleaseBufferBatch(arr, len(handles))


def _shape_size(shape):
    s = 1
    for d in shape:
        s *= d
    return s


# --------------------------------------------------------------------------
# Tensor / Function
# --------------------------------------------------------------------------
# Every buffer this module creates goes through _create_buffer, so that
# discover_buffer_sizes can watch the sizes a training step asks for.
_size_log = None


def _create_buffer(ptr, count):
    if _size_log is not None:
        _size_log.add(int(count))
    return lib.CreateBuffer(ptr, count)


def _fptr(arr):
    return arr.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Tensor:
    """A device buffer handle with a shape and an autograd context.

    `data` is the host array the tensor was built from, or the array that
    sync() last filled; device work never updates it by itself."""
    __slots__ = ["data", "shape", "size", "requires_grad", "grad", "gpu_buf", "_ctx", "_cached_topo"]

    def __init__(self, data, requires_grad=False, track=True):
        arr = data if isinstance(data, np.ndarray) else np.array(data, dtype=np.float32)
        if arr.dtype != np.float32:
            arr = arr.astype(np.float32)
        arr = np.ascontiguousarray(arr)
        self._init_fields(arr.shape, requires_grad, _create_buffer(_fptr(arr), arr.size), track)
        self.data = arr

    def _init_fields(self, shape, requires_grad, handle, track):
        self.data = None
        self.shape = shape
        self.size = _shape_size(shape)
        self.requires_grad = requires_grad
        self.grad = None
        self.gpu_buf = handle
        self._ctx = None
        if track:
            _all_tensors.append(self)

    def __del__(self):
        try:
            h, self.gpu_buf = self.gpu_buf, None
            if h:
                lib.ReleaseBuffer(h)
        except Exception:
            pass

    @classmethod
    def from_gpu(cls, handle, shape, requires_grad=False, track=True):
        """Wrap an existing handle (ownership moves to the tensor)."""
        t = object.__new__(cls)
        t._init_fields(shape, requires_grad, handle, track)
        return t

    @classmethod
    def empty(cls, shape, requires_grad=False, track=True):
        """A tensor over a pooled buffer whose contents are undefined."""
        shape = tuple(shape)
        h = _check(_create_buffer(None, _shape_size(shape)), "CreateBuffer")
        return cls.from_gpu(h, shape, requires_grad=requires_grad, track=track)

    @classmethod
    def empty_like(cls, other, requires_grad=None, track=True):
        req = other.requires_grad if requires_grad is None else bool(requires_grad)
        return cls.empty(other.shape, requires_grad=req, track=track)

    def sync(self):
        """Blocking read-back into self.data (allocated on first use)."""
        if not self.gpu_buf:
            return self.data
        want = tuple(self.shape)
        if self.data is None or self.data.shape != want:
            self.data = np.empty(want, dtype=np.float32)
        lib.ReadBuffer(self.gpu_buf, _fptr(self.data))
        return self.data

    def upload(self, data):
        """Overwrite the device buffer with `data` (no new buffer)."""
        arr = np.ascontiguousarray(data, dtype=np.float32)
        self.data, self.shape, self.size = arr, arr.shape, arr.size
        lib.UpdateBuffer(self.gpu_buf, _fptr(arr))

    def _topo_order(self):
        """Every tensor that takes part in the backward pass, each after all of
        its inputs.  Depth-first post-order from this tensor in which a node's
        inputs are taken last to first: the order nn_engine.py:575-603
        produces, which fixes the order gradients are accumulated in."""
        order, done = [], set()
        frames = [[self, None]]           # [node, inputs still to take]
        while frames:
            frame = frames[-1]
            node = frame[0]
            if frame[1] is None:
                if node in done:
                    frames.pop()
                    continue
                ins = node._ctx.inputs if node._ctx else ()
                frame[1] = [t for t in ins if isinstance(t, Tensor) and t.requires_grad]
            todo = frame[1]
            while todo and todo[-1] in done:
                todo.pop()
            if todo:
                frames.append([todo.pop(), None])
            else:
                done.add(node)
                order.append(node)
                frames.pop()
        return order

    def backward(self, grad=None):
        """Seed this tensor's gradient (ones by default) and run every
        Function.backward from the output towards the leaves.  The traversal
        order is computed once per output tensor and cached."""
        self.grad = grad if grad is not None else Tensor(np.ones(self.shape, np.float32), track=False)
        try:
            order = self._cached_topo
        except AttributeError:
            order = self._cached_topo = self._topo_order()
        for node in reversed(order):
            ctx = node._ctx
            if ctx and node.grad is not None:
                ctx.backward(node.grad)

    def _accumulate_grad(self, grad):
        """First gradient is aliased; later ones are added in place with
        grad_accum (nn_engine.py:605-610)."""
        if self.grad is None or self.grad.gpu_buf is None:
            self.grad = grad
        else:
            _dispatch(b"grad_accum", (grad.gpu_buf,), (self.grad.gpu_buf,),
                      (self.size + 255) // 256, 1, 1, u1=self.size)


class Function:
    def __init__(self, *inputs):
        self.inputs = inputs

    def backward(self, grad_output):
        raise NotImplementedError


def _new(count, what):
    return _check(_create_buffer(None, count), what)


# Flagged GEMM into a caller's buffer.  The reference chooses its shader by
# output size; here every flagged-GEMM name reaches the same MFMA GEMM (the
# launch shape comes from the constants), so the choice only keeps the shader
# names of a recorded dispatch the same.
_MM_SMALL_TILE, _MM_LARGE_TILE, _MM_LARGE_MIN = 16, 64, 64


def _run_mm(a_buf, b_buf, out_buf, M, K, N, flags=0):
    """out = op(A)·op(B) into an existing buffer of M×N floats (flags bit0: A
    stored K×M, bit1: B stored N×K), the helper the reference's matmul
    benchmarks and verification scripts call (nn_engine.py:887-893)."""
    large = M >= _MM_LARGE_MIN and N >= _MM_LARGE_MIN
    t = _MM_LARGE_TILE if large else _MM_SMALL_TILE
    _dispatch(b"matmul_dgpu" if large else b"matmul_universal", (a_buf, b_buf), (out_buf,),
              (N + t - 1) // t, (M + t - 1) // t, 1, u1=M, u2=K, u3=N, u4=flags)


# --------------------------------------------------------------------------
# Ops
# --------------------------------------------------------------------------
class MatMul(Function):
    """Y = op(A)·op(B) via MatMulAlloc; backward computes dA/dB straight into
    the raw layouts of A/B for the four transpose combinations
    (nn_engine.py:913-952)."""

    def forward(self, A, B, transA=False, transB=False):
        self.inputs = (A, B)
        self.transA, self.transB = transA, transB
        self.A_shape, self.B_shape = A.shape, B.shape
        flags = (1 if transA else 0) | (2 if transB else 0)
        M = A.shape[1] if transA else A.shape[0]
        K = A.shape[0] if transA else A.shape[1]
        N = B.shape[0] if transB else B.shape[1]
        h = _check(lib.MatMulAlloc(A.gpu_buf, B.gpu_buf, M, K, N, flags), "MatMulAlloc")
        res = Tensor.from_gpu(h, (M, N), requires_grad=A.requires_grad or B.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        A, B = self.inputs
        a0, a1 = self.A_shape
        b0, b1 = self.B_shape
        M, N = grad_output.shape
        g = grad_output.gpu_buf
        tA, tB = self.transA, self.transB
        if A.requires_grad:
            if not tA and not tB:
                h = lib.MatMulAlloc(g, B.gpu_buf, M, N, a1, 2)      # dY·Bᵀ
            elif not tA and tB:
                h = lib.MatMulAlloc(g, B.gpu_buf, M, N, b1, 0)      # dY·B
            elif tA and not tB:
                h = lib.MatMulAlloc(B.gpu_buf, g, a0, N, a1, 2)     # B·dYᵀ
            else:
                h = lib.MatMulAlloc(B.gpu_buf, g, a0, N, a1, 3)     # Bᵀ·dYᵀ
            A._accumulate_grad(Tensor.from_gpu(_check(h, "MatMul.backward(dA)"), A.shape, track=True))
        if B.requires_grad:
            if not tA and not tB:
                h = lib.MatMulAlloc(A.gpu_buf, g, a1, a0, N, 1)     # Aᵀ·dY
            elif not tA and tB:
                h = lib.MatMulAlloc(g, A.gpu_buf, b0, a0, a1, 1)    # dYᵀ·A
            elif tA and not tB:
                h = lib.MatMulAlloc(A.gpu_buf, g, a0, a1, b1, 0)    # A·dY
            else:
                h = lib.MatMulAlloc(g, A.gpu_buf, b0, a1, b1, 3)    # dYᵀ·Aᵀ
            B._accumulate_grad(Tensor.from_gpu(_check(h, "MatMul.backward(dB)"), B.shape, track=True))


class Conv2D(Function):
    """ConvForwardFused / ConvBackwardFused (nn_engine.py:954-1016).  The
    implicit-GEMM library keeps no im2col matrix: `im2col_handle` holds the
    forward's channel-innermost copy of x (the stride-phase or channel-packed
    copy for fewer than 4 input channels, a 4-float placeholder for pointwise
    layers), which ConvBackwardFused consumes and releases."""

    def __del__(self):
        h = getattr(self, "im2col_handle", None)
        if h:
            try:
                lib.ReleaseBuffer(h)
            except Exception:
                pass
            self.im2col_handle = None

    def forward(self, x, filters, bias, stride=1, padding=0, actType=0):
        self.inputs = (x, filters, bias)
        self.stride, self.padding, self.actType = stride, padding, actType
        batch, inC, inH, inW = x.shape
        outC, _, kH, kW = filters.shape
        outH = (inH + 2 * padding - kH) // stride + 1
        outW = (inW + 2 * padding - kW) // stride + 1
        needs_backward = x.requires_grad or filters.requires_grad or bias.requires_grad
        p_im2col = ctypes.c_void_p()
        h = lib.ConvForwardFused(x.gpu_buf, filters.gpu_buf, bias.gpu_buf, batch, inC, inH, inW,
                                 outC, kH, kW, stride, padding, actType,
                                 ctypes.byref(p_im2col) if needs_backward else None)
        _check(h, "ConvForwardFused")
        self.im2col_handle = p_im2col.value if needs_backward else None
        res = Tensor.from_gpu(h, (batch, outC, outH, outW), requires_grad=needs_backward)
        self.fwd_output = res if actType != 0 and needs_backward else None
        res._ctx = self
        return res

    def backward(self, grad_output):
        x, filters, bias = self.inputs
        batch, inC, inH, inW = x.shape
        outC, _, kH, kW = filters.shape
        pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        fwd = self.fwd_output.gpu_buf if self.fwd_output else None
        lib.ConvBackwardFused(grad_output.gpu_buf, fwd, x.gpu_buf, filters.gpu_buf,
                              self.im2col_handle, batch, inC, inH, inW, outC, kH, kW,
                              self.stride, self.padding, self.actType,
                              1 if x.requires_grad else 0, 1 if filters.requires_grad else 0,
                              1 if bias.requires_grad else 0,
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
        self.fwd_output = None
        self.im2col_handle = None  # consumed by ConvBackwardFused
        if (filters.requires_grad and not pdf.value) or (x.requires_grad and not pdx.value):
            raise RuntimeError(f"ConvBackwardFused failed: {last_error()}")
        if pdf.value:
            filters._accumulate_grad(Tensor.from_gpu(pdf.value, filters.shape, track=True))
        if pdb.value:
            bias._accumulate_grad(Tensor.from_gpu(pdb.value, bias.shape, track=True))
        if pdx.value:
            x._accumulate_grad(Tensor.from_gpu(pdx.value, x.shape, track=True))


class MaxPool2D(Function):
    def __del__(self):
        h = getattr(self, "indices_handle", None)
        if h:
            try:
                lib.ReleaseBuffer(h)
            except Exception:
                pass
            self.indices_handle = None

    def forward(self, x, pool_size=2, stride=2):
        self.inputs = (x,)
        batch, inC, inH, inW = x.shape
        outH = (inH - pool_size) // stride + 1
        outW = (inW - pool_size) // stride + 1
        p_idx = ctypes.c_void_p()
        h = _check(lib.MaxPoolForwardFused(x.gpu_buf, batch, inC, inH, inW, pool_size, stride,
                                           ctypes.byref(p_idx)), "MaxPoolForwardFused")
        self.indices_handle = p_idx.value
        res = Tensor.from_gpu(h, (batch, inC, outH, outW), requires_grad=x.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        x = self.inputs[0]
        batch, inC, outH, outW = grad_output.shape
        h = lib.MaxPoolBackwardFused(grad_output.gpu_buf, self.indices_handle, batch, inC, outH,
                                     outW, x.size)
        self.indices_handle = None  # consumed by MaxPoolBackwardFused
        x._accumulate_grad(Tensor.from_gpu(_check(h, "MaxPoolBackwardFused"), x.shape, track=True))


class Flatten(Function):
    def forward(self, x):
        self.inputs = (x,)
        lib.AddRefBuffer(x.gpu_buf)
        res = Tensor.from_gpu(x.gpu_buf, (x.shape[0], x.size // x.shape[0]),
                              requires_grad=x.requires_grad, track=False)
        res._ctx = self
        return res

    def backward(self, grad_output):
        lib.AddRefBuffer(grad_output.gpu_buf)
        self.inputs[0]._accumulate_grad(
            Tensor.from_gpu(grad_output.gpu_buf, self.inputs[0].shape, track=False))


def _bias_grad(g_tensor, rows, n):
    h = _new(n, "bias_grad")
    _dispatch(b"bias_grad", (g_tensor.gpu_buf,), (h,), n, 1, 1, u1=rows, u2=n, u3=n, u4=1)
    return h


class AddBias(Function):
    def forward(self, A, B):
        self.inputs = (A, B)
        h = _new(A.size, "add_bias")
        _dispatch(b"add_bias", (A.gpu_buf, B.gpu_buf), (h,), (A.size + 255) // 256, 1, 1,
                  u1=A.shape[0], u2=A.shape[1])
        res = Tensor.from_gpu(h, A.shape, requires_grad=A.requires_grad or B.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        A, B = self.inputs
        if A.requires_grad:
            A._accumulate_grad(grad_output)
        if B.requires_grad:
            B._accumulate_grad(Tensor.from_gpu(_bias_grad(grad_output, grad_output.shape[0], B.size),
                                               B.shape, track=True))


class BiasReLUFunc(Function):
    """add_bias + ReLU; backward masks on the *output* (nn_engine.py:1091-1106)."""

    def forward(self, A, B):
        self.inputs = (A, B)
        h = _new(A.size, "bias_relu")
        _dispatch(b"bias_relu", (A.gpu_buf, B.gpu_buf), (h,), (A.size + 255) // 256, 1, 1,
                  u1=A.shape[0], u2=A.shape[1])
        res = Tensor.from_gpu(h, A.shape, requires_grad=A.requires_grad or B.requires_grad)
        self.output = res
        res._ctx = self
        return res

    def backward(self, grad_output):
        A, B = self.inputs
        out = self.output
        h = _new(grad_output.size, "relu_grad")
        _dispatch(b"relu_grad", (grad_output.gpu_buf, out.gpu_buf), (h,),
                  (grad_output.size + 255) // 256, 1, 1, u1=grad_output.size)
        eff = Tensor.from_gpu(h, grad_output.shape, track=True)
        self.output = None
        if A.requires_grad:
            A._accumulate_grad(eff)
        if B.requires_grad:
            B._accumulate_grad(Tensor.from_gpu(_bias_grad(eff, eff.shape[0], B.size), B.shape, track=True))


class _Unary(Function):
    """Elementwise op y = f(x) whose backward shader reads (grad, saved)."""
    fwd_name = None
    bwd_name = None
    save_output = False

    def _cb(self, x):
        return dict(u1=x.size)

    def forward(self, x):
        self.inputs = (x,)
        h = _new(x.size, self.fwd_name.decode())
        if self.fwd_name == b"relu":
            _dispatch(b"relu", (x.gpu_buf,), (h,), (x.size + 255) // 256, 1, 1, cbSize=0)
        else:
            _dispatch(self.fwd_name, (x.gpu_buf,), (h,), (x.size + 255) // 256, 1, 1, **self._cb(x))
        res = Tensor.from_gpu(h, x.shape, requires_grad=x.requires_grad)
        res._ctx = self
        if self.save_output:
            self.out_tensor = res
        return res

    def backward(self, grad_output):
        x = self.inputs[0]
        if x.requires_grad:
            saved = self.out_tensor if self.save_output else x
            h = _new(x.size, self.bwd_name.decode())
            _dispatch(self.bwd_name, (grad_output.gpu_buf, saved.gpu_buf), (h,),
                      (x.size + 255) // 256, 1, 1, **self._cb(x))
            x._accumulate_grad(Tensor.from_gpu(h, x.shape, track=True))


class ReLUFunc(_Unary):
    fwd_name, bwd_name = b"relu", b"relu_grad"


class ReLU6Func(_Unary):
    fwd_name, bwd_name = b"relu6", b"relu6_grad"


class SigmoidFunc(_Unary):
    fwd_name, bwd_name, save_output = b"sigmoid", b"sigmoid_grad", True


class LeakyReLUFunc(_Unary):
    fwd_name, bwd_name = b"leaky_relu", b"leaky_relu_grad"

    def forward(self, x, alpha=0.1):
        self.alpha = alpha
        return super().forward(x)

    def _cb(self, x):
        return dict(u1=x.size, u2=float_to_uint(self.alpha))


class UpSample2D(Function):
    def forward(self, x, scaleH=2, scaleW=2):
        self.inputs = (x,)
        self.scaleH, self.scaleW = scaleH, scaleW
        batch, C, inH, inW = x.shape
        outH, outW = inH * scaleH, inW * scaleW
        n = batch * C * outH * outW
        h = _new(n, "upsample")
        _dispatch(b"upsample", (x.gpu_buf,), (h,), (n + 255) // 256, 1, 1, u1=batch, u2=C, u3=inH,
                  u4=inW, u5=outH, u6=outW, u7=scaleH, u8=scaleW, cbSize=32)
        res = Tensor.from_gpu(h, (batch, C, outH, outW), requires_grad=x.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        x = self.inputs[0]
        if x.requires_grad:
            batch, C, inH, inW = x.shape
            h = _new(x.size, "upsample_backward")
            _dispatch(b"upsample_backward", (grad_output.gpu_buf,), (h,), (x.size + 255) // 256, 1, 1,
                      u1=batch, u2=C, u3=inH, u4=inW, u5=inH * self.scaleH, u6=inW * self.scaleW,
                      u7=self.scaleH, u8=self.scaleW, cbSize=32)
            x._accumulate_grad(Tensor.from_gpu(h, x.shape, track=True))


class Concat(Function):
    def forward(self, tensors, axis=1):
        if axis != 1:
            raise NotImplementedError("Concat currently only supported along channel dimension (axis 1)")
        self.inputs = tuple(tensors)
        batch, H, W = tensors[0].shape[0], tensors[0].shape[2], tensors[0].shape[3]
        S = H * W
        total_C = sum(t.shape[1] for t in tensors)
        h = _new(batch * total_C * S, "concat")
        off = 0
        self.c_offsets = []
        for t in tensors:
            self.c_offsets.append(off)
            c_in = t.shape[1]
            n = batch * c_in * S
            _dispatch(b"concat_insert", (t.gpu_buf,), (h,), (n + 255) // 256, 1, 1, u1=batch, u2=c_in,
                      u3=S, u4=total_C, u5=off, cbSize=20)
            off += c_in
        res = Tensor.from_gpu(h, (batch, total_C, H, W), requires_grad=any(t.requires_grad for t in tensors))
        res._ctx = self
        return res

    def backward(self, grad_output):
        batch, total_C, H, W = grad_output.shape
        S = H * W
        for t, off in zip(self.inputs, self.c_offsets):
            if t.requires_grad:
                c_in = t.shape[1]
                n = batch * c_in * S
                h = _new(n, "slice")
                _dispatch(b"slice", (grad_output.gpu_buf,), (h,), (n + 255) // 256, 1, 1, u1=batch,
                          u2=c_in, u3=S, u4=total_C, u5=off, cbSize=20)
                t._accumulate_grad(Tensor.from_gpu(h, t.shape, track=True))


class SoftmaxCEFunc(Function):
    """softmax + mean CE loss; backward (p - onehot)/B ignoring the incoming
    gradient (nn_engine.py:1268-1288)."""

    def forward(self, x, labels):
        self.inputs = (x, labels)
        B, K = x.shape
        hs = _new(x.size, "softmax")
        _dispatch(b"softmax", (x.gpu_buf,), (hs,), (B + 15) // 16, 1, 1, u1=B, u2=K)
        self.softmax_out = Tensor.from_gpu(hs, x.shape)
        hl = _new(1, "loss")
        _dispatch(b"loss", (x.gpu_buf, labels.gpu_buf), (hl,), 1, 1, 1, u1=B, u2=K)
        res = Tensor.from_gpu(hl, (1,), requires_grad=True)
        res._ctx = self
        return res

    def backward(self, grad_output):
        x, labels = self.inputs
        B, K = x.shape
        h = _new(x.size, "softmax_ce_grad")
        _dispatch(b"softmax_ce_grad", (self.softmax_out.gpu_buf, labels.gpu_buf), (h,),
                  (K + 15) // 16, (B + 15) // 16, 1, u1=B, u2=K)
        x._accumulate_grad(Tensor.from_gpu(h, x.shape, track=True))


class DiceLossFunc(Function):
    def forward(self, pred, target):
        self.inputs = (pred, target)
        batch = pred.shape[0]
        size = pred.size // batch
        h = _new(batch, "dice_loss")
        _dispatch(b"dice_loss", (pred.gpu_buf, target.gpu_buf), (h,), batch, 1, 1, u1=batch, u2=size)
        res = Tensor.from_gpu(h, (batch,), requires_grad=True)
        res._ctx = self
        return res

    def backward(self, grad_output):
        pred, target = self.inputs
        batch = pred.shape[0]
        size = pred.size // batch
        hs = _new(batch * 3, "dice_loss_sums")
        _dispatch(b"dice_loss_sums", (pred.gpu_buf, target.gpu_buf), (hs,), batch, 1, 1, u1=batch, u2=size)
        h = _new(pred.size, "dice_loss_grad")
        _dispatch(b"dice_loss_grad", (pred.gpu_buf, target.gpu_buf, hs), (h,), (pred.size + 255) // 256,
                  1, 1, u1=batch, u2=size)
        lib.ReleaseBuffer(hs)
        pred._accumulate_grad(Tensor.from_gpu(h, pred.shape, track=True))


class AddFunc(Function):
    """Residual add; backward passes the same buffer to both inputs via
    AddRef (nn_engine.py:1379-1397)."""

    def forward(self, A, B):
        self.inputs = (A, B)
        h = _new(A.size, "add")
        _dispatch(b"add", (A.gpu_buf, B.gpu_buf), (h,), (A.size + 255) // 256, 1, 1, u1=A.size, u2=1)
        res = Tensor.from_gpu(h, A.shape, requires_grad=A.requires_grad or B.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        A, B = self.inputs
        for t in (A, B):
            if t.requires_grad:
                lib.AddRefBuffer(grad_output.gpu_buf)
                t._accumulate_grad(Tensor.from_gpu(grad_output.gpu_buf, t.shape, track=False))


class DepthwiseConv2DFunc(Function):
    def forward(self, x, filters, bias, stride=1, padding=0):
        self.inputs = (x, filters, bias)
        self.stride, self.padding = stride, padding
        batch, C, inH, inW = x.shape
        kH, kW = filters.shape[2], filters.shape[3]
        outH = (inH + 2 * padding - kH) // stride + 1
        outW = (inW + 2 * padding - kW) // stride + 1
        n = batch * C * outH * outW
        h = _new(n, "depthwise_conv_forward")
        _dispatch(b"depthwise_conv_forward", (x.gpu_buf, filters.gpu_buf, bias.gpu_buf), (h,),
                  (n + 255) // 256, 1, 1, u1=batch, u2=C, u3=inH, u4=inW, u5=kH, u6=kW, u7=stride,
                  u8=padding, u9=outH, cbSize=36)
        res = Tensor.from_gpu(h, (batch, C, outH, outW),
                              requires_grad=x.requires_grad or filters.requires_grad or bias.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        x, filters, bias = self.inputs
        batch, C, inH, inW = x.shape
        kH, kW = filters.shape[2], filters.shape[3]
        outH = grad_output.shape[2]
        cb = dict(u1=batch, u2=C, u3=inH, u4=inW, u5=kH, u6=kW, u7=self.stride, u8=self.padding,
                  u9=outH, cbSize=36)
        if x.requires_grad:
            h = _new(x.size, "depthwise_conv_backward_input")
            _dispatch(b"depthwise_conv_backward_input", (grad_output.gpu_buf, filters.gpu_buf), (h,),
                      (x.size + 255) // 256, 1, 1, **cb)
            x._accumulate_grad(Tensor.from_gpu(h, x.shape, track=True))
        if filters.requires_grad or bias.requires_grad:
            hf = _new(filters.size, "depthwise dW")
            hb = _new(bias.size, "depthwise db")
            _dispatch(b"depthwise_conv_backward_filter", (grad_output.gpu_buf, x.gpu_buf), (hf, hb),
                      C, 1, 1, **cb)
            if filters.requires_grad:
                filters._accumulate_grad(Tensor.from_gpu(hf, filters.shape, track=True))
            else:
                lib.ReleaseBuffer(hf)
            if bias.requires_grad:
                bias._accumulate_grad(Tensor.from_gpu(hb, bias.shape, track=True))
            else:
                lib.ReleaseBuffer(hb)


class GlobalAvgPool2DFunc(Function):
    def forward(self, x):
        self.inputs = (x,)
        batch, C, H, W = x.shape
        self.S = H * W
        h = _new(batch * C, "global_avg_pool")
        _dispatch(b"global_avg_pool", (x.gpu_buf,), (h,), batch * C, 1, 1, u1=batch, u2=C, u3=self.S)
        res = Tensor.from_gpu(h, (batch, C), requires_grad=x.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        x = self.inputs[0]
        if x.requires_grad:
            batch, C = grad_output.shape
            h = _new(x.size, "global_avg_pool_backward")
            _dispatch(b"global_avg_pool_backward", (grad_output.gpu_buf,), (h,), (x.size + 255) // 256,
                      1, 1, u1=batch, u2=C, u3=self.S)
            x._accumulate_grad(Tensor.from_gpu(h, x.shape, track=True))


class BatchNorm2dFunc(Function):
    """Training-mode BN: batchnorm_mean_var + batchnorm_forward; backward
    batchnorm_backward_reduce then batchnorm_backward_dx (nn_engine.py:1794-1868)."""

    def forward(self, x, gamma, beta, running_mean, running_var, eps=1e-5, momentum=0.1, training=True):
        self.inputs = (x, gamma, beta)
        self.batch, self.channels, self.h, self.w = x.shape
        self.S = self.h * self.w
        self.eps = eps
        if training:
            self.batch_mean_handle = _new(self.channels, "bn mean")
            self.batch_var_handle = _new(self.channels, "bn var")
            _dispatch(b"batchnorm_mean_var", (x.gpu_buf,),
                      (self.batch_mean_handle, self.batch_var_handle, running_mean.gpu_buf, running_var.gpu_buf),
                      self.channels, 1, 1, u1=self.batch, u2=self.channels, u3=self.S, u4=1,
                      u5=float_to_uint(momentum), cbSize=20)
            mean_buf, var_buf = self.batch_mean_handle, self.batch_var_handle
        else:
            mean_buf, var_buf = running_mean.gpu_buf, running_var.gpu_buf
            self.batch_mean_handle = self.batch_var_handle = None
        h = _new(x.size, "batchnorm_forward")
        _dispatch(b"batchnorm_forward", (x.gpu_buf, mean_buf, var_buf, gamma.gpu_buf, beta.gpu_buf), (h,),
                  (x.size + 255) // 256, 1, 1, u1=self.batch, u2=self.channels, u3=self.S,
                  u4=float_to_uint(eps), cbSize=16)
        res = Tensor.from_gpu(h, x.shape, requires_grad=x.requires_grad or gamma.requires_grad or beta.requires_grad)
        res._ctx = self
        return res

    def backward(self, grad_output):
        x, gamma, beta = self.inputs
        if self.batch_mean_handle is None:
            raise RuntimeError("BatchNorm backward requires training=True during forward")
        hg = _new(self.channels, "bn dgamma")
        hb = _new(self.channels, "bn dbeta")
        cb = dict(u1=self.batch, u2=self.channels, u3=self.S, u4=float_to_uint(self.eps))
        _dispatch(b"batchnorm_backward_reduce",
                  (x.gpu_buf, grad_output.gpu_buf, self.batch_mean_handle, self.batch_var_handle),
                  (hg, hb), self.channels, 1, 1, **cb)
        hx = _new(x.size, "bn dx")
        _dispatch(b"batchnorm_backward_dx",
                  (x.gpu_buf, grad_output.gpu_buf, self.batch_mean_handle, self.batch_var_handle,
                   gamma.gpu_buf, hg, hb), (hx,), (x.size + 255) // 256, 1, 1, **cb)
        for t, h in ((gamma, hg), (beta, hb), (x, hx)):
            if t.requires_grad:
                t._accumulate_grad(Tensor.from_gpu(h, t.shape, track=True))
            else:
                lib.ReleaseBuffer(h)
        lib.ReleaseBuffer(self.batch_mean_handle)
        lib.ReleaseBuffer(self.batch_var_handle)
        self.batch_mean_handle = self.batch_var_handle = None


def _absent(name):
    def f(*args, **kwargs):
        raise NotImplementedError(f"{name}: its kernels do not exist in the reference tree "
                                  "(nn_engine.py:156-163 names shaders with no source)")
    return f


gelu = _absent("gelu")
layernorm = _absent("layernorm")
attention = _absent("attention")


def matmul(A, B, transA=False, transB=False): return MatMul().forward(A, B, transA, transB)
def add_bias(A, B): return AddBias().forward(A, B)
def bias_relu(A, B): return BiasReLUFunc().forward(A, B)
def relu(x): return ReLUFunc().forward(x)
def relu6(x): return ReLU6Func().forward(x)
def sigmoid(x): return SigmoidFunc().forward(x)
def softmax_ce(x, labels): return SoftmaxCEFunc().forward(x, labels)
def conv2d(x, f, b, stride=1, padding=0, actType=0): return Conv2D().forward(x, f, b, stride, padding, actType)
def maxpool2d(x, pool_size=2, stride=2): return MaxPool2D().forward(x, pool_size, stride)
def flatten(x): return Flatten().forward(x)
def leaky_relu(x, alpha=0.1): return LeakyReLUFunc().forward(x, alpha)
def upsample2d(x, scaleH=2, scaleW=2): return UpSample2D().forward(x, scaleH, scaleW)
def concat(tensors, axis=1): return Concat().forward(tensors, axis)
def dice_loss(pred, target): return DiceLossFunc().forward(pred, target)
def add(A, B): return AddFunc().forward(A, B)
def depthwise_conv2d(x, f, b, stride=1, padding=0): return DepthwiseConv2DFunc().forward(x, f, b, stride, padding)
def global_avg_pool2d(x): return GlobalAvgPool2DFunc().forward(x)


def batchnorm2d(x, gamma, beta, rm, rv, eps=1e-5, momentum=0.1, training=True):
    return BatchNorm2dFunc().forward(x, gamma, beta, rm, rv, eps, momentum, training)


def _handle_arrays(params):
    n = len(params)
    pa = (ctypes.c_void_p * n)(*[p.gpu_buf for p in params])
    ga = (ctypes.c_void_p * n)(*[(p.grad.gpu_buf if p.grad is not None else None) for p in params])
    sa = (ctypes.c_uint * n)(*[p.size for p in params])
    return pa, ga, sa


def clip_grad_norm(params, max_norm=1.0):
    """Global L2 norm of all gradients; when it exceeds max_norm every gradient
    is scaled by max_norm/(norm+1e-6).  Returns the norm (nn_engine.py:1335-1355).
    Computed on the GPU (one multi-tensor reduction + one scale pass); only the
    norm is read back."""
    live = [p for p in params if p.grad is not None and p.grad.gpu_buf is not None]
    if not live:
        return 0.0
    n = len(live)
    ga = (ctypes.c_void_p * n)(*[p.grad.gpu_buf for p in live])
    sa = (ctypes.c_uint * n)(*[p.size for p in live])
    return float(lib.ClipGradNorm(ga, sa, n, max_norm))


def sgd_step_clipped(params, lr, max_norm=1.0):
    """Fused norm clip + SGD on the GPU; returns the norm (nn_engine.py:1357-1367)."""
    pa, ga, sa = _handle_arrays(params)
    return float(lib.SGDBatchClipped(pa, ga, sa, len(params), lr, max_norm))


def scale_add(A, B, alpha=1.0, beta=1.0):
    h = _new(A.size, "scale_add")
    _dispatch(b"scale_add", (A.gpu_buf, B.gpu_buf), (h,), (A.size + 255) // 256, 1, 1, u1=A.size,
              u2=float_to_uint(alpha), u3=float_to_uint(beta), cbSize=16)
    return Tensor.from_gpu(h, A.shape, track=True)


# --------------------------------------------------------------------------
# Layers and Model (initialisers as nn_engine.py:1873-1927)
# --------------------------------------------------------------------------
class Linear:
    def __init__(self, in_features, out_features):
        limit = np.sqrt(6 / (in_features + out_features))
        self.w = Tensor(np.random.uniform(-limit, limit, (in_features, out_features)), requires_grad=True, track=False)
        self.b = Tensor(np.zeros(out_features), requires_grad=True, track=False)

    def __call__(self, x, relu=False):
        m = matmul(x, self.w)
        return bias_relu(m, self.b) if relu else add_bias(m, self.b)


class ConvLayer:
    def __init__(self, inC, outC, ks, stride=1, padding=0):
        fan_in, fan_out = inC * ks * ks, outC * ks * ks
        limit = np.sqrt(6 / (fan_in + fan_out))
        self.filters = Tensor(np.random.uniform(-limit, limit, (outC, inC, ks, ks)), requires_grad=True, track=False)
        self.bias = Tensor(np.zeros(outC), requires_grad=True, track=False)
        self.stride, self.padding = stride, padding

    def __call__(self, x, actType=0, relu=False):
        return conv2d(x, self.filters, self.bias, self.stride, self.padding, 1 if relu else actType)


class DepthwiseConvLayer:
    def __init__(self, channels, ks, stride=1, padding=0):
        limit = np.sqrt(6 / (ks * ks * 2))
        self.filters = Tensor(np.random.uniform(-limit, limit, (channels, 1, ks, ks)), requires_grad=True, track=False)
        self.bias = Tensor(np.zeros(channels), requires_grad=True, track=False)
        self.stride, self.padding = stride, padding

    def __call__(self, x):
        return depthwise_conv2d(x, self.filters, self.bias, self.stride, self.padding)


class BatchNorm2d:
    def __init__(self, num_features, eps=1e-5, momentum=0.1):
        self.num_features = num_features
        self.eps, self.momentum = eps, momentum
        self.gamma = Tensor(np.ones(num_features, dtype=np.float32), requires_grad=True, track=False)
        self.beta = Tensor(np.zeros(num_features, dtype=np.float32), requires_grad=True, track=False)
        self.running_mean = Tensor(np.zeros(num_features, dtype=np.float32), requires_grad=False, track=False)
        self.running_var = Tensor(np.ones(num_features, dtype=np.float32), requires_grad=False, track=False)
        self.training = True

    def __call__(self, x):
        return batchnorm2d(x, self.gamma, self.beta, self.running_mean, self.running_var, self.eps,
                           self.momentum, self.training)


def _param_attrs(obj):
    """Attributes holding a layer's trainable tensors, in the order
    Model.parameters lists them.  Normalisation layers are matched by class
    name, so that a model's own BatchNorm2d / LayerNorm classes count too
    (nn_engine.py:1959-1971)."""
    if isinstance(obj, (ConvLayer, DepthwiseConvLayer)):
        return ("filters", "bias")
    if isinstance(obj, Linear):
        return ("w", "b")
    if type(obj).__name__ in ("BatchNorm2d", "LayerNorm"):
        return ("gamma", "beta")
    return ()


class Model:
    """Base class of user models: parameter discovery, train / eval mode.

    Layers are found among the model's attributes in dir() order (sorted by
    name), as in nn_engine.py:1930-1987."""

    def __init__(self):
        self._forward_trace = []

    def __call__(self, x):
        return self.forward(x)

    def forward(self, x):
        raise NotImplementedError

    def _members(self):
        return ((name, getattr(self, name)) for name in dir(self))

    def parameters(self):
        return [getattr(layer, a) for _, layer in self._members() for a in _param_attrs(layer)]

    def train(self, mode=True):
        for _, member in self._members():
            if hasattr(member, "training"):
                member.training = mode

    def eval(self):
        self.train(False)

    def _get_layers(self):
        kinds = (ConvLayer, DepthwiseConvLayer, Linear)
        return [(n, m) for n, m in self._members() if isinstance(m, kinds)]


# --------------------------------------------------------------------------
# Optimisers (nn_engine.py:2172-2242)
# --------------------------------------------------------------------------
# True while ComputeGraph records a step: the optimiser then records work
# that stays valid on every replay (AdamW advances its device step counter
# instead of setting it).
_recording = False


class _Optimizer:
    """Parameters, zero_grad, and the handle tables a multi-tensor launch
    takes (allocated once; refilled each step with the parameters that have a
    gradient)."""

    def __init__(self, params, lr):
        self.params = params
        self.lr = lr
        n = len(params)
        self._pa = (ctypes.c_void_p * n)()
        self._ga = (ctypes.c_void_p * n)()
        self._sa = (ctypes.c_uint * n)()

    def zero_grad(self):
        for p in self.params:
            p.grad = None

    def _live(self):
        """Fill the tables with (param, grad, size) of every parameter that has
        a gradient, in parameter order; returns their indices."""
        live = [i for i, p in enumerate(self.params) if p.grad is not None]
        for slot, i in enumerate(live):
            p = self.params[i]
            self._pa[slot], self._ga[slot], self._sa[slot] = p.gpu_buf, p.grad.gpu_buf, p.size
        return live


class SGD(_Optimizer):
    def step(self, clip=1.0):
        """w -= lr*clamp(g, -clip, clip) for every parameter with a gradient."""
        n = len(self._live())
        if n:
            lib.SGDBatch(self._pa, self._ga, self._sa, n, self.lr, clip)


class AdamW(_Optimizer):
    """AdamW with the reference's update rule: bias-corrected step size
    lr*sqrt(1-b2^t)/(1-b1^t), decay lr*wd*w on the old weight, element clip of
    the gradient; one multi-tensor launch per step.  The step count lives on
    the device too (AdamBatchCounted), so that a step recorded by ComputeGraph
    replays as the next step; `t` mirrors it on the host."""

    def __init__(self, params, lr=0.001, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01):
        super().__init__(params, lr)
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.weight_decay = weight_decay
        self.t = 0
        self.m = [Tensor(np.zeros(p.shape, np.float32), track=False) for p in params]
        self.v = [Tensor(np.zeros(p.shape, np.float32), track=False) for p in params]
        self._state = Tensor(np.zeros(2, np.float32), track=False)  # [t bits, step size]
        n = len(params)
        self._ma = (ctypes.c_void_p * n)()
        self._va = (ctypes.c_void_p * n)()

    def step(self, clip=1.0):
        self.t += 1
        # bias-corrected step size, evaluated as nn_engine.py:2220 does; a
        # recorded step (t argument 0) has the device evaluate it per replay
        step_size = self.lr * (1 - self.beta2 ** self.t) ** 0.5 / (1 - self.beta1 ** self.t)
        live = self._live()
        for slot, i in enumerate(live):
            self._ma[slot], self._va[slot] = self.m[i].gpu_buf, self.v[i].gpu_buf
        if live:
            lib.AdamBatchCounted(self._pa, self._ga, self._ma, self._va, self._sa, len(live),
                                 self._state.gpu_buf, 0 if _recording else self.t, step_size,
                                 self.lr, self.beta1, self.beta2, self.eps,
                                 self.lr * self.weight_decay, clip)


class Adam(AdamW):
    def __init__(self, params, lr=0.001, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        super().__init__(params, lr, betas, eps, weight_decay=weight_decay)


# --------------------------------------------------------------------------
# Metrics, batch end, pool helpers (nn_engine.py:2322-2485)
# --------------------------------------------------------------------------
def gpu_argmax_correct(logits, labels, correct_buf):
    batch_size, num_classes = logits.shape
    _dispatch_raw(b"argmax_correct", (logits.gpu_buf, labels.gpu_buf), (correct_buf,),
                  (batch_size + 255) // 256, 1, 1, u1=batch_size, u2=num_classes)


def gpu_accumulate_loss(loss_tensor, accum_buf):
    _dispatch(b"accumulate_scalar", (loss_tensor.gpu_buf,), (accum_buf,), 1, 1, 1, cbSize=0)


class Metrics:
    """Loss and accuracy accumulated on the device over an epoch; collect()
    is the only read-back (nn_engine.py:2336-2385).  The correct count is a
    u32 held in a float buffer."""

    def __init__(self):
        self._bufs = {"loss": _new(1, "Metrics"), "correct": _new(1, "Metrics")}
        self._host = np.zeros(1, np.float32)
        self._n_batches = 0
        self.reset()

    def reset(self):
        for h in self._bufs.values():
            lib.ClearBuffer(h)
        self._n_batches = 0

    def update(self, loss, logits, labels):
        gpu_accumulate_loss(loss, self._bufs["loss"])
        gpu_argmax_correct(logits, labels, self._bufs["correct"])
        self._n_batches += 1

    def _read(self, key):
        lib.ReadBuffer(self._bufs[key], _fptr(self._host))
        return self._host.copy()

    def collect(self, num_samples):
        """(mean loss per batch, accuracy over num_samples)."""
        total = float(self._read("loss")[0])
        correct = int(self._read("correct").view(np.uint32)[0])
        mean_loss = total / self._n_batches if self._n_batches else 0.0
        return mean_loss, (correct / num_samples if num_samples else 0.0)

    def __del__(self):
        try:
            bufs, self._bufs = self._bufs, {}
            for h in bufs.values():
                lib.ReleaseBuffer(h)
        except Exception:
            pass


def end_batch():
    """Release the batch's intermediates; FlushGPU every flush_interval batches."""
    release_all_buffers()
    end_batch._count += 1
    if end_batch._count % end_batch.flush_interval == 0:
        lib.FlushGPU()


end_batch._count = 0
end_batch.flush_interval = 10


class ComputeGraph:
    """Record one training step -- forward, loss, backward, optional global
    norm clip and the optimiser update -- once, then replay it with new data
    (nn_engine.py:2505-2771).

    The reference records the step's RunShader dispatches and replays them with
    RunSequence plus an SGDBatch call, so the fused conv / pool / matmul calls
    fall outside its record.  Here the library captures every launch of the
    step on its stream as a HIP graph (BeginCapture / EndCapture): any model
    replays, with one ReplayGraph call per batch, and the graph holds the
    step's buffers until release().

    trace() runs the traced batch eagerly (which also sizes the pool and the
    workspace), then records the same step.  The loss is softmax-CE unless
    `loss_fn(logits, labels)` is given (e.g. dice_loss); `max_norm` adds the
    global gradient-norm clip before the update (clip_grad_norm, computed and
    applied on the device).  Host scalars are those of the recorded step (SGD
    learning rate and clip); Adam / AdamW keep their step count on the device,
    so every replay is the next step, and `optimizer.t` follows the replays.
    The step may not read buffers back or upload more than 256 floats.
    """

    def __init__(self):
        self._graph = None
        self._handles = {}         # input, labels, loss, logits
        self._shapes = {}
        self._optimizer = None
        self._compiled = False

    def _step(self, forward_fn, optimizer, clip, loss_fn, max_norm, params):
        optimizer.zero_grad()
        wrapped = {}
        for key in ("input", "labels"):
            lib.AddRefBuffer(self._handles[key])
            # The traced input's gradient is never readable after the step, so
            # it is not requested (nn_engine.py:2631 asks for it and drops it).
            wrapped[key] = Tensor.from_gpu(self._handles[key], self._shapes[key])
        logits = forward_fn(wrapped["input"])
        loss = (loss_fn or softmax_ce)(logits, wrapped["labels"])
        loss.backward()
        if max_norm is not None:
            clip_grad_norm(params, max_norm)
        optimizer.step(clip=clip)
        return loss, logits

    def _keep(self, key, tensor):
        lib.AddRefBuffer(tensor.gpu_buf)
        self._handles[key] = tensor.gpu_buf
        self._shapes[key] = tuple(tensor.shape)

    def _upload(self, key, arr):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        if a.shape != self._shapes[key]:
            raise ValueError(f"replay {key} shape {a.shape} differs from the traced {self._shapes[key]}")
        lib.UpdateBuffer(self._handles[key], _fptr(a))

    def trace(self, forward_fn, optimizer, X_batch, Y_batch, params, clip=1.0, loss_fn=None,
              max_norm=None):
        """Run one batch eagerly, then record the same step as a graph.
        Returns the eager step's (loss, logits) tensors, whose buffers are
        released on return as in the reference."""
        self.release()
        for key, arr in (("input", X_batch), ("labels", Y_batch)):
            a = np.ascontiguousarray(arr, dtype=np.float32)
            self._handles[key] = _check(_create_buffer(_fptr(a), a.size), "CreateBuffer")
            self._shapes[key] = a.shape
        step_args = (forward_fn, optimizer, clip, loss_fn, max_norm, params)
        loss, logits = self._step(*step_args)
        eager = {"loss": loss.sync().copy(), "logits": logits.sync().copy()}
        release_all_buffers()

        global _recording
        t_before = getattr(optimizer, "t", None)
        if not lib.BeginCapture():
            raise RuntimeError(f"BeginCapture failed: {last_error()}")
        _recording = True
        try:
            rec_loss, rec_logits = self._step(*step_args)
            self._keep("loss", rec_loss)
            self._keep("logits", rec_logits)
        except BaseException:
            _recording = False
            graph = lib.EndCapture()
            release_all_buffers()
            if graph:
                lib.ReleaseGraph(graph)
            self.release()
            raise
        finally:
            _recording = False
            if t_before is not None:
                optimizer.t = t_before   # the recorded step has not run yet
        graph = lib.EndCapture()
        release_all_buffers()
        if not graph:
            self.release()
            raise RuntimeError(f"ComputeGraph.trace: capture failed: {last_error()}")
        self._graph = graph
        self._optimizer = optimizer
        self._params_ref = params
        self._compiled = True
        # read_loss / read_logits before the first replay give the eager step's values
        for key in ("loss", "logits"):
            lib.UpdateBuffer(self._handles[key], _fptr(eager[key]))
        return loss, logits

    def replay(self, X_batch=None, Y_batch=None):
        """Upload a new batch into the traced input / label buffers and enqueue
        one replay of the step.  A batch given as None is not uploaded: the
        step then runs on what the buffer holds (the last batch, or data a
        caller wrote into input_tensor() / label_tensor() on the device)."""
        if not self._compiled:
            raise RuntimeError("Graph not compiled. Call trace() first.")
        if X_batch is not None:
            self._upload("input", X_batch)
        if Y_batch is not None:
            self._upload("labels", Y_batch)
        if not lib.ReplayGraph(self._graph):
            raise RuntimeError(f"ReplayGraph failed: {last_error()}")
        if hasattr(self._optimizer, "t"):
            self._optimizer.t += 1

    def _read(self, key):
        out = np.empty(self._shapes[key], dtype=np.float32)
        lib.ReadBuffer(self._handles[key], _fptr(out))
        return out

    def read_loss(self):
        """The last step's loss (the mean, for a per-sample loss such as Dice)."""
        v = self._read("loss")
        return float(v.reshape(-1)[0]) if v.size == 1 else float(v.mean())

    def read_logits(self):
        return self._read("logits")

    def _view(self, key):
        lib.AddRefBuffer(self._handles[key])
        return Tensor.from_gpu(self._handles[key], self._shapes[key], track=False)

    def input_tensor(self):
        """The traced input buffer as a tensor (a new reference), so that a
        batch already on the device can be copied in without a host trip."""
        return self._view("input")

    def label_tensor(self):
        return self._view("labels")

    def release(self):
        """Free the graph, the buffers it holds and the input / label buffers."""
        if self._graph:
            lib.ReleaseGraph(self._graph)
            self._graph = None
        handles, self._handles = self._handles, {}
        for h in handles.values():
            if h:
                lib.ReleaseBuffer(h)
        self._compiled = False

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


def warm_pool(sizes, copies=2):
    """Pre-allocate `copies` pooled buffers of every element count in `sizes`."""
    counts = sorted(int(c) for c in sizes)
    lib.WarmPool((ctypes.c_uint * len(counts))(*counts), len(counts), copies)


def discover_buffer_sizes(forward_fn, params, X_batch, Y_batch, optimizer):
    """Element counts of the buffers one softmax-CE training step creates from
    Python (nn_engine.py:2421-2444): the step runs once, eagerly, with the
    module's buffer-creation hook recording every count."""
    global _size_log
    seen = set()
    _size_log = seen
    try:
        optimizer.zero_grad()
        logits = forward_fn(Tensor(X_batch, track=True))
        softmax_ce(logits, Tensor(Y_batch, track=True)).backward()
        optimizer.step(clip=1.0)
        end_batch()
    finally:
        _size_log = None
    return seen


def auto_warm(forward_fn, params, X_sample, Y_sample, optimizer, copies=2):
    """discover_buffer_sizes, then warm_pool with those counts; the pool's
    hit / miss counters restart afterwards."""
    found = discover_buffer_sizes(forward_fn, params, X_sample, Y_sample, optimizer)
    warm_pool(found, copies)
    lib.ResetPoolStats()
    return found


def get_pool_stats():
    hits, misses = ctypes.c_uint64(0), ctypes.c_uint64(0)
    lib.GetPoolStats(ctypes.byref(hits), ctypes.byref(misses))
    return hits.value, misses.value


def get_pool_memory():
    return lib.GetPoolMemory()


def drain_pool():
    lib.DrainPool()


def sync_gpu():
    """Block until all queued GPU work is done."""
    lib.SyncGPU()


# --------------------------------------------------------------------------
# Profiler
# --------------------------------------------------------------------------
class KernelProfiler:
    """The reference's `profiler` object (nn_engine.py:183-306) with the same
    calls -- install / uninstall / enable / disable / reset / report -- but
    measured on the device: the engine brackets each kernel family's launches
    with HIP events on its stream, so `report` shows GPU time per family (the
    reference times the host-side ctypes calls, which on an asynchronous
    stream measure submission).  Nothing is wrapped, so install() and
    uninstall() have nothing to do.  The memory lines report the buffer
    pool: bytes held for reuse and its hit / miss counts."""

    # Families the engine records: the fused paths and every RunShader
    # kernel that runs under its own name.
    FAMILIES = ("conv_fwd", "conv_bwd", "conv_dw", "conv_dx", "gemm", "nhwc", "conv_grad_nhwc",
                "maxpool_fwd", "maxpool_bwd", "bn_stats", "bn_stats_side", "bn_fwd", "bn_bwd_reduce",
                "bn_bwd_reduce_side", "bn_bwd_dx",
                "dw_bwd_input", "dw_bwd_filter", "gap_bwd", "upsample", "upsample_bwd", "bias_grad",
                "dice_loss_grad", "sgd", "sgd_clipped", "adam", "grad_norm", "clip_scale",
                "relu", "relu_grad", "relu6", "relu6_grad", "leaky_relu", "leaky_relu_grad",
                "sigmoid", "sigmoid_grad", "add", "scale_add", "grad_accum")

    def __init__(self):
        self.enabled = False

    def install(self):
        pass

    def uninstall(self):
        pass

    def enable(self):
        self.enabled = True
        lib.SetProfiling(1)
        self.reset()

    def disable(self):
        self.enabled = False
        lib.SetProfiling(0)

    def reset(self):
        lib.ResetProfile()
        lib.ResetPoolStats()

    def stats(self):
        """{family: (launches, total ms)} recorded since the last reset."""
        lib.SyncGPU()
        out = {}
        n, ms = ctypes.c_uint64(), ctypes.c_double()
        fl, by = ctypes.c_double(), ctypes.c_double()
        for f in self.FAMILIES:
            if lib.GetProfile(f.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl),
                              ctypes.byref(by)) and n.value:
                out[f] = (int(n.value), float(ms.value))
        return out

    # Families that enclose others: conv_bwd brackets each whole
    # ConvBackwardFused call, whose conv_dw, conv_dx and conv_grad_nhwc
    # launches are recorded under their own names as well.
    AGGREGATES = ("conv_bwd",)

    @classmethod
    def table(cls, st):
        """Rows (family, calls, ms, % of time) of the leaf families, the
        aggregate rows (family, calls, ms) and the leaf total (calls, ms).
        Aggregates are left out of the total, so the percentages add up to
        100 and no time is counted twice."""
        leaf = {f: v for f, v in st.items() if f not in cls.AGGREGATES}
        total = sum(ms for _, ms in leaf.values())
        calls = sum(c for c, _ in leaf.values())
        rows = [(f, c, ms, 100.0 * ms / total if total else 0.0)
                for f, (c, ms) in sorted(leaf.items(), key=lambda kv: -kv[1][1])]
        aggs = [(f, *st[f]) for f in cls.AGGREGATES if f in st]
        return rows, aggs, (calls, total)

    def report(self, epoch_label=""):
        if not self.enabled:
            return
        rows, aggs, (calls, total) = self.table(self.stats())
        bar = "=" * 80
        print(f"\n{bar}\n  GPU kernel time {epoch_label}\n{bar}")
        print(f"  {'Family':<28} {'Calls':>6} {'Total ms':>10} {'Avg ms':>10} {'% Time':>8}")
        for f, c, ms, pct in rows:
            print(f"  {f:<28} {c:>6} {ms:>10.3f} {ms / c:>10.4f} {pct:>7.1f}%")
        print(f"  {'TOTAL':<28} {calls:>6} {total:>10.3f}")
        for f, c, ms in aggs:
            print(f"  {f + ' (whole calls, in TOTAL)':<28} {c:>6} {ms:>10.3f} {ms / c:>10.4f}")
        hits, misses = get_pool_stats()
        print(f"\n  Pool held:  {get_pool_memory() / 1024 / 1024:>8.2f} MB  "
              f"(requests: {hits} reused, {misses} allocated)\n{bar}\n")


profiler = KernelProfiler()
