"""ctypes front end of tests/ort_double/libxm_ort_double.so: the custom-op
layer registered into the ONNX Runtime API double and run node by node, as
an ONNX Runtime session would (kernel from node attributes, Compute on bound
tensors).  Tensors are NumPy arrays (host) or torch tensors (device); output
buffers are bound by the caller and viewed with the shapes the kernel asked
for.  Test infrastructure only."""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "ort_double", "libxm_ort_double.so")

FLOAT, INT64, FLOAT16, BFLOAT16 = 1, 7, 10, 16
REQUIRED, OPTIONAL = 0, 1


class Tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("shape", ctypes.c_int64 * 8), ("rank", ctypes.c_int32),
                ("elem_type", ctypes.c_int32), ("present", ctypes.c_int32), ("device", ctypes.c_int32),
                ("capacity", ctypes.c_uint64)]


_lib = None


def lib():
    """The double, built beforehand (tests/ort_double/build.py; the CPU tests
    build it when it is missing)."""
    global _lib
    if _lib is None:
        import xmetai_onnx_plugins as xp
        xp.lib()   # the operator library (and torch's HIP runtime) first
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built: python tests/ort_double/build.py")
        l = ctypes.CDLL(LIB)
        l.ortd_register.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
        l.ortd_register_with_nulls.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]
        l.ortd_register_with_max_version.argtypes = [ctypes.c_uint32, ctypes.c_char_p, ctypes.c_size_t,
                                                     ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        l.ortd_requested_api_version.restype = ctypes.c_uint32
        l.ortd_domain_name.restype = ctypes.c_char_p
        l.ortd_op_name.restype = ctypes.c_char_p
        l.ortd_op_ep.restype = ctypes.c_char_p
        l.ortd_op_version.restype = ctypes.c_uint32
        l.ortd_op_slot.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        l.ortd_run.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                               ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                               ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.POINTER(Tensor), ctypes.c_int,
                               ctypes.POINTER(Tensor), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                               ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int), ctypes.c_char_p,
                               ctypes.c_size_t]
        err = ctypes.create_string_buffer(512)
        if l.ortd_register(err, len(err)) != 0:
            raise RuntimeError("RegisterCustomOps failed: " + err.value.decode())
        _lib = l
    return _lib


def ops():
    """[(domain, name, execution provider, inputs, outputs)], inputs/outputs
    being [(element type, characteristic)], in registration order."""
    l = lib()
    out = []
    for d in range(l.ortd_domain_count()):
        dom = l.ortd_domain_name(d).decode()
        for i in range(l.ortd_op_count(d)):
            slots = []
            for o in (0, 1):
                s = []
                for k in range(l.ortd_op_arity(d, i, o)):
                    t, c = ctypes.c_int(), ctypes.c_int()
                    l.ortd_op_slot(d, i, o, k, ctypes.byref(t), ctypes.byref(c))
                    s.append((t.value, c.value))
                slots.append(s)
            out.append((dom, l.ortd_op_name(d, i).decode(), l.ortd_op_ep(d, i).decode(), slots[0], slots[1]))
    return out


def find(name, input0_type=FLOAT):
    """(domain, index) of the descriptor a session would bind a node to: by
    name and the element type of input 0."""
    for idx, (_, n, _, ins, _) in enumerate(ops()):
        if n == name and ins[0][0] == input0_type:
            return 0, idx
    raise KeyError((name, input0_type))


def _elem(x):
    import numpy as np
    if x is None:
        return 0
    if isinstance(x, np.ndarray):
        return {np.dtype(np.float32): FLOAT, np.dtype(np.int64): INT64, np.dtype(np.float16): FLOAT16}.get(x.dtype, 0)
    import torch
    return {torch.float32: FLOAT, torch.int64: INT64, torch.float16: FLOAT16, torch.bfloat16: BFLOAT16}.get(x.dtype, 0)


def _bind(x, capacity=False):
    t = Tensor()
    if x is None:
        t.present = 0
        t.rank = 0
        return t
    import numpy as np
    t.present = 1
    if isinstance(x, np.ndarray):
        t.data = x.ctypes.data if x.size else None
        t.device = 0
        nbytes = x.nbytes
    else:
        t.data = x.data_ptr() if x.numel() else None
        t.device = 1 if x.is_cuda else 0
        nbytes = x.numel() * x.element_size()
    t.rank = x.ndim
    for d, n in enumerate(x.shape):
        t.shape[d] = n
    t.elem_type = _elem(x)
    if capacity:
        t.capacity = nbytes
    return t


class RunError(RuntimeError):
    def __init__(self, stage, msg):
        super().__init__(f"{stage}: {msg}")
        self.stage, self.msg = stage, msg


def run(name, inputs, outputs, ints=None, floats=None, stream=None, scratch=None, input0_type=None):
    """One node: returns the outputs viewed with the shapes the kernel asked
    for (None where it did not write), plus (scratch high-water mark, scratch
    buffers freed).  Raises RunError('create' | 'compute', message)."""
    l = lib()
    ints, floats = dict(ints or {}), dict(floats or {})
    d, i = find(name, input0_type if input0_type is not None else (_elem(inputs[0]) or FLOAT))
    ins = (Tensor * max(1, len(inputs)))(*[_bind(x) for x in inputs])
    outs = (Tensor * max(1, len(outputs)))(*[_bind(x, capacity=True) for x in outputs])
    inames = (ctypes.c_char_p * max(1, len(ints)))(*[k.encode() for k in ints])
    ivals = (ctypes.c_int64 * max(1, len(ints)))(*ints.values())
    fnames = (ctypes.c_char_p * max(1, len(floats)))(*[k.encode() for k in floats])
    fvals = (ctypes.c_float * max(1, len(floats)))(*floats.values())
    sp, sbytes = None, 0
    if scratch is not None:
        sp, sbytes = scratch.data_ptr(), scratch.numel() * scratch.element_size()
    peak, frees = ctypes.c_uint64(), ctypes.c_int()
    err = ctypes.create_string_buffer(1024)
    rc = l.ortd_run(d, i, len(ints), inames, ivals, len(floats), fnames, fvals, len(inputs), ins, len(outputs),
                    outs, stream, sp, sbytes, ctypes.byref(peak), ctypes.byref(frees), err, len(err))
    if rc == 1:
        raise RunError("create", err.value.decode())
    if rc != 0:
        raise RunError("compute", err.value.decode())
    res = []
    for k, x in enumerate(outputs):
        t = outs[k]
        if not t.present:
            res.append(None)
            continue
        shape = tuple(t.shape[j] for j in range(t.rank))
        n = 1
        for s in shape:
            n *= s
        res.append(x.reshape(-1)[:n].reshape(shape))
    return res, (peak.value, frees.value)
