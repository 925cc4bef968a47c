"""MI355X (gfx950) recurrent operators of the ONNX domain ``xmetai_plugins``.

Python front end of ``libxmetai_recurrent.so`` (C ABI in
``include/xmetai_recurrent.h``).  The three functions take the operators'
inputs in the reference's order, as fp32 torch tensors on a ROCm device, and
enqueue the HIP kernels on the current torch stream:

* :func:`selective_scan_fn`   -- ``SelectiveScanFn``  (selective_scan_fn_ort.cpp:48-246)
* :func:`mamba3_siso_fn`      -- ``Mamba3SisoFn``     (mamba3_siso_fn_ort.cpp:41-246)
* :func:`gated_deltanet2_fn`  -- ``GatedDeltaNet2Fn`` (gated_deltanet2_fn_ort.cpp:44-237)

"Optional" inputs are passed as ``None`` or a zero-element tensor, exactly as
the ONNX graphs pass them (every input of the reference ops is REQUIRED; an
empty tensor means absent).  Errors raise :class:`XmError` carrying the C
status code and the reference's message.  There is no CPU fallback: without
the built library, or without a GPU, the forward functions raise.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Sequence

from . import _capi
from ._capi import (XM_ERR_ALLOC, XM_ERR_DEVICE, XM_ERR_INVALID_ARGUMENT, XM_ERR_UNSUPPORTED, XM_OK,
                    EXPORTED_SYMBOLS, LIB_PATH)

__all__ = [
    "XmError", "PreparedCall", "lib", "version", "last_launches", "set_kernel_override", "get_kernel_override", "kernel_override", "selective_scan_fn", "mamba3_siso_fn", "gated_deltanet2_fn", "softmax_cpu",
    "validate", "TorchAllocator", "EXPORTED_SYMBOLS", "LIB_PATH",
    "XM_OK", "XM_ERR_INVALID_ARGUMENT", "XM_ERR_UNSUPPORTED", "XM_ERR_DEVICE", "XM_ERR_ALLOC",
]

DOMAIN = "xmetai_plugins"
# registration order of the reference (register_op.cpp:24-39)
OP_NAMES = ("SelectiveScanFn", "Mamba3SisoFn", "GatedDeltaNet2Fn", "SoftmaxCPU")

_lib = None


class XmError(RuntimeError):
    """An error status returned by the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{_capi.STATUS_NAMES.get(status, status)}] {message}")
        self.status = status
        self.message = message


def lib() -> ctypes.CDLL:
    """Loads the in-tree library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python xmetai-onnx-plugins_amd/build.py` "
                "(there is no fallback implementation)")
        # torch wheels carry their own HIP runtime (torch/lib/libamdhip64.so).
        # Import torch first so the library binds to that runtime; loaded
        # before it, the library would pull in /opt/rocm's libamdhip64 and the
        # process would hold two runtimes whose streams and device pointers do
        # not mix (every launch then fails with hipErrorNoDevice).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        _lib = _capi.declare(ctypes.CDLL(LIB_PATH))
    return _lib


def version() -> str:
    return lib().xm_version().decode()


def last_launches() -> list:
    """Kernels this thread's last operator call enqueued (names as rocprofv3
    prints them, with " xN" for repeated launches)."""
    s = lib().xm_last_launches().decode()
    return s.split(";") if s else []


def set_kernel_override(name: str, value: int) -> None:
    """Forces a kernel variant process-wide (tests and tuning); 0 restores the
    dispatcher's choice.  Names and values: ``_capi.KERNEL_OVERRIDES``."""
    err = ctypes.create_string_buffer(256)
    _check(lib().xm_set_kernel_override(name.encode(), int(value), err, len(err)), err)


def get_kernel_override(name: str) -> int:
    return int(lib().xm_get_kernel_override(name.encode()))


class kernel_override:
    """Context manager: ``with kernel_override("m3_path", 1): ...`` restores the
    previous value on exit."""

    def __init__(self, name: str, value: int):
        self.name, self.value, self.prev = name, value, None

    def __enter__(self):
        self.prev = get_kernel_override(self.name)
        set_kernel_override(self.name, self.value)
        return self

    def __exit__(self, *exc):
        set_kernel_override(self.name, self.prev)
        return False


# ---------------------------------------------------------------------------
# tensor descriptors
# ---------------------------------------------------------------------------

_DUMMY = ctypes.c_void_p(16)  # non-null address for shape-only validation; never dereferenced


def _desc_from_shape(shape: Sequence[int], data_ptr: Optional[int] = None, elem_type: int = 1) -> _capi.XmTensor:
    t = _capi.XmTensor()
    if len(shape) > _capi.XM_MAX_RANK:
        raise XmError(XM_ERR_INVALID_ARGUMENT, "tensor rank out of range")
    t.rank = len(shape)
    for i, d in enumerate(shape):
        t.shape[i] = int(d)
    t.elem_type = elem_type
    n = math.prod(int(d) for d in shape) if len(shape) else 1
    if data_ptr is not None:
        t.data = data_ptr
    else:
        t.data = _DUMMY.value if n > 0 else None
    return t


def _desc_from_tensor(x) -> _capi.XmTensor:
    import torch
    if x is None:
        return _desc_from_shape((0,))
    if not isinstance(x, torch.Tensor):
        raise TypeError("inputs must be torch tensors or None")
    elem = {torch.float32: _capi.XM_ELEM_FLOAT, torch.int64: _capi.XM_ELEM_INT64,
            torch.float16: _capi.XM_ELEM_FLOAT16, torch.bfloat16: _capi.XM_ELEM_BFLOAT16}.get(x.dtype, 0)
    if x.numel() > 0:
        if not x.is_cuda:
            raise XmError(XM_ERR_INVALID_ARGUMENT, "inputs must be device tensors")
        if not x.is_contiguous():
            raise XmError(XM_ERR_INVALID_ARGUMENT, "inputs must be contiguous (row-major)")
    return _desc_from_shape(tuple(x.shape), x.data_ptr() if x.numel() > 0 else None, elem)


def _attrs(op: str, **kw):
    attrs_t, _ = _capi.OPS[op]
    a = attrs_t()
    getattr(lib(), f"xm_{op}_attrs_default")(ctypes.byref(a))
    for k, v in kw.items():
        if v is None:
            continue
        if not hasattr(a, k):
            raise TypeError(f"unknown attribute {k} for {op}")
        setattr(a, k, float(v) if k == "scale" else int(v))
    return a


def _check(status: int, err: ctypes.Array) -> None:
    if status != XM_OK:
        raise XmError(status, err.value.decode(errors="replace"))


def validate(op: str, shapes: Sequence[Optional[Sequence[int]]], elem_types: Optional[Sequence[int]] = None,
             **attrs):
    """Runs the operator's host-side validation on shapes only (no device).

    ``op`` is ``"selective_scan"``, ``"mamba3_siso"`` or ``"gated_deltanet2"``;
    ``shapes`` lists one shape per input (``None`` = absent); ``elem_types``
    one ONNX element type per input (default float; cu_seqlens is int64).
    Returns ``(output_shape, scratch_bytes)`` or raises :class:`XmError`.
    """
    _, n = _capi.OPS[op]
    counts = {n}
    if op == "mamba3_siso":
        counts |= {_capi.MAMBA3_INPUTS_WITH_STATES, _capi.MAMBA3_INPUTS_PACKED}
    if op == "gated_deltanet2":
        counts |= {_capi.GDN2_INPUTS_PACKED}
    if len(shapes) not in counts:
        raise TypeError(f"{op} takes {n} inputs")
    n = len(shapes)
    types = list(elem_types) if elem_types is not None else [_capi.XM_ELEM_FLOAT] * n
    arr = (_capi.XmTensor * n)(*[_desc_from_shape(s if s is not None else (0,), elem_type=e)
                                 for s, e in zip(shapes, types)])
    a = _attrs(op, **attrs)
    out_shape = (ctypes.c_int64 * _capi.XM_MAX_RANK)()
    out_rank = ctypes.c_int32()
    scratch = ctypes.c_size_t()
    err = ctypes.create_string_buffer(512)
    st = getattr(lib(), f"xm_{op}_validate")(arr, n, ctypes.byref(a), out_shape, ctypes.byref(out_rank),
                                             ctypes.byref(scratch), err, len(err))
    _check(st, err)
    return tuple(out_shape[i] for i in range(out_rank.value)), scratch.value


def check_attrs(op: str, **attrs) -> None:
    """Session-time attribute checks (the reference's kernel constructors)."""
    a = _attrs(op, **attrs)
    err = ctypes.create_string_buffer(512)
    _check(getattr(lib(), f"xm_{op}_check_attrs")(ctypes.byref(a), err, len(err)), err)


# ---------------------------------------------------------------------------
# allocator over torch's caching allocator (stream-ordered)
# ---------------------------------------------------------------------------

class TorchAllocator:
    """Scratch from torch's caching allocator on a given stream.

    torch reuses a freed block only in the order of the stream it was
    allocated on, which is the stream the operator runs on, so returning the
    block right after the launches is safe (the contract of xm_allocator_t).
    """

    def __init__(self, device=None, stream=None):
        import torch
        self._torch = torch
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.stream = stream
        self.live = 0

        def _alloc(ctx, nbytes):
            s = self.stream if self.stream is not None else torch.cuda.current_stream(self.device)
            try:
                ptr = torch.cuda.caching_allocator_alloc(int(nbytes), self.device.index, s)
            except Exception:
                return None
            self.live += 1
            return ptr

        def _free(ctx, ptr):
            if ptr:
                torch.cuda.caching_allocator_delete(ptr)
                self.live -= 1

        self._alloc_cb = _capi.ALLOC_FN(_alloc)
        self._free_cb = _capi.FREE_FN(_free)
        self.struct = _capi.XmAllocator(None, self._alloc_cb, self._free_cb)


# ---------------------------------------------------------------------------
# operators
# ---------------------------------------------------------------------------

class PreparedCall:
    """One operator call whose argument blocks are built once (``prepare=True``
    on the operator functions).  Calling it enqueues the same forward again:
    the same input, output and state buffers, on the stream it was prepared
    for, through the same C entry point.  It skips the per-call work of the
    plain functions (tensor descriptors, attribute blocks, output allocation),
    which is most of the host time of a small call.  The caller keeps the
    inputs alive; ``out`` and ``states`` are overwritten by every call, and a
    call returns what the operator function would have."""

    def __init__(self, fn, args, err, keep, device_index, out, states, result):
        self._fn = fn
        self._args = args
        self._err = err
        self._keep = keep
        self._device_index = device_index
        self.out = out
        self.states = states
        self._result = result

    def __call__(self):
        import torch
        if torch.cuda.current_device() != self._device_index:
            with torch.cuda.device(self._device_index):
                st = self._fn(*self._args)
        else:
            st = self._fn(*self._args)
        _check(st, self._err)
        return self._result


def _run(op: str, inputs, out_like_index: int, allocator: Optional[TorchAllocator], stream,
         state_shapes=None, prepare=False, **attrs):
    """Validates and enqueues one operator call.  With ``state_shapes`` (one
    shape per state buffer) set it calls the op's ``_forward_states`` entry
    point and returns ``(out, [state, ...])``.  With ``prepare`` it enqueues
    nothing and returns a :class:`PreparedCall` instead."""
    import torch
    n = len(inputs)
    descs = [_desc_from_tensor(x) for x in inputs]
    arr = (_capi.XmTensor * n)(*descs)
    a = _attrs(op, **attrs)
    err = ctypes.create_string_buffer(512)
    out_shape = (ctypes.c_int64 * _capi.XM_MAX_RANK)()
    out_rank = ctypes.c_int32()
    scratch = ctypes.c_size_t()
    _check(getattr(lib(), f"xm_{op}_validate")(arr, n, ctypes.byref(a), out_shape, ctypes.byref(out_rank),
                                               ctypes.byref(scratch), err, len(err)), err)
    ref = inputs[out_like_index]
    # SelectiveScanFn's y takes u's element type (fp32, or the 16-bit data types)
    out_dtype = ref.dtype if op == "selective_scan" else torch.float32
    out = torch.empty(tuple(out_shape[i] for i in range(out_rank.value)), dtype=out_dtype, device=ref.device)
    if stream is None:
        stream = torch.cuda.current_stream(ref.device)
    alloc_ptr = ctypes.byref(allocator.struct) if allocator is not None else None
    out_ptr = ctypes.c_void_p(out.data_ptr() if out.numel() else None)
    stream_ptr = ctypes.c_void_p(stream.cuda_stream)
    if state_shapes is None:
        fn = getattr(lib(), f"xm_{op}_forward")
        args = (arr, n, ctypes.byref(a), out_ptr, stream_ptr, alloc_ptr, err, len(err))
        states, result = None, out
    else:
        states = [torch.empty(tuple(int(d) for d in sh), dtype=torch.float32, device=ref.device)
                  for sh in state_shapes]
        fn = getattr(lib(), f"xm_{op}_forward_states")
        args = (arr, n, ctypes.byref(a), out_ptr,
                *(ctypes.c_void_p(x.data_ptr() if x.numel() else None) for x in states),
                stream_ptr, alloc_ptr, err, len(err))
        result = (out, states)
    if prepare:
        keep = (inputs, arr, a, allocator, stream)
        return PreparedCall(fn, args, err, keep, ref.device.index, out, states, result)
    with torch.cuda.device(ref.device):
        st = fn(*args)
    _check(st, err)
    return result


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, *, delta_softplus=False,
                      return_last_state=False, allocator=None, stream=None, prepare=False):
    """SelectiveScanFn: returns y [B,D,L] (the un-gated scan output; z is
    validated and otherwise unused, as in selective_scan_fwd_kernel.cuh:272-301).

    With ``return_last_state=True`` (rejected by the reference's ORT kernel,
    selective_scan_fn_ort.cpp:52-55; accepted here as a widening) it returns
    ``(y, last_state)``, last_state [B,D,N] being the scan state after the
    last token (zeros when L = 0).

    u, delta, z and variable B/C may be float16 or bfloat16 (all the same;
    the reference's half / bfloat16 kernels, unreachable from its fp32 host):
    A, D, delta_bias and constant B/C stay float32, y takes u's type and the
    state stays float32.  ``prepare=True`` returns a :class:`PreparedCall`
    (same for the other operators)."""
    shapes = None   # shapes of other ranks fail validation before the launch
    if return_last_state and u.dim() == 3 and A.dim() == 2:
        shapes = [(u.shape[0], u.shape[1], A.shape[1])]
    r = _run("selective_scan", [u, delta, A, B, C, D, z, delta_bias], 0, allocator, stream,
             state_shapes=shapes, prepare=prepare,
             delta_softplus=int(bool(delta_softplus)), return_last_state=int(bool(return_last_state)))
    if prepare:
        if shapes is not None:
            r._result = (r.out, r.states[0])
        return r
    return (r[0], r[1][0]) if shapes is not None else r


def mamba3_siso_fn(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D=None, Z=None, *, chunk_size=64,
                   has_d=None, has_z=None, input_states=None, return_final_states=False, has_input_states=None,
                   cu_seqlens=None, allocator=None, stream=None, prepare=False):
    """Mamba3SisoFn: returns [B,T,H,P].  ``has_d``/``has_z`` default to the
    presence of D/Z (an exported graph sets them explicitly; default 1).

    States (rejected by the reference, mamba3_siso_fn_ort.cpp:50-55; accepted
    here as a widening): ``input_states`` = (ssm [B,H,P,N], angle [B,H,A],
    k [B,H,N], v [B,H,P]) continues a previous call; ``return_final_states``
    returns ``(y, (ssm, angle, k, v))`` after the last token.

    Packed sequences (rejected by the reference, :56-58): ``cu_seqlens`` (int64
    [N+1] device tensor) splits the single row of tokens (batch 1) into N
    sequences; the states are then [N, ...], one per sequence."""
    def present(x):
        return x is not None and x.numel() > 0
    has_d = present(D) if has_d is None else has_d
    has_z = present(Z) if has_z is None else has_z
    has_input_states = input_states is not None if has_input_states is None else has_input_states
    inputs = [Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z]
    if has_input_states:
        inputs += list(input_states)
    elif cu_seqlens is not None:
        inputs += [None] * 4   # the state slots before cu_seqlens
    if cu_seqlens is not None:
        inputs.append(cu_seqlens)
    shapes = None   # shapes of other ranks fail validation before the launch
    if return_final_states and Q.dim() == 4 and V.dim() == 4 and Angles.dim() == 4:
        b = cu_seqlens.shape[0] - 1 if cu_seqlens is not None else Q.shape[0]
        h, pdim, n, a = V.shape[2], V.shape[3], Q.shape[3], Angles.shape[3]
        shapes = [(b, h, pdim, n), (b, h, a), (b, h, n), (b, h, pdim)]
    r = _run("mamba3_siso", inputs, 2, allocator, stream, state_shapes=shapes, prepare=prepare,
             chunk_size=chunk_size, has_d=int(bool(has_d)), has_z=int(bool(has_z)),
             return_final_states=int(bool(return_final_states)), has_input_states=int(bool(has_input_states)),
             has_cu_seqlens=int(cu_seqlens is not None))
    if prepare:
        if shapes is not None:
            r._result = (r.out, tuple(r.states))
        return r
    return (r[0], tuple(r[1])) if shapes is not None else r


def gated_deltanet2_fn(q, k, v, g, beta, w, initial_state=None, *, scale=1.0, use_qk_l2norm_in_kernel=True,
                       output_final_state=False, use_gate_in_kernel=False, cu_seqlens=None,
                       state_v_first=False, allocator=None, stream=None, prepare=False):
    """GatedDeltaNet2Fn: returns [B,T,H,V].

    With ``output_final_state=True`` (rejected by the reference,
    gated_deltanet2_fn_ort.cpp:49-51; accepted here as a widening) it returns
    ``(o, final_state)``, final_state [B,H,K,V] being the state after the last
    token in initial_state's layout.

    Packed sequences (rejected by the reference, gated_deltanet2_fn_ort.cpp:55-57):
    ``cu_seqlens`` (int64 [N+1] device tensor) splits the single row of tokens
    (batch 1) into N sequences; initial_state and final_state are then [N,H,K,V]."""
    shapes = None   # shapes of other ranks fail validation before the launch
    if output_final_state and q.dim() == 4 and v.dim() == 4:
        n = cu_seqlens.shape[0] - 1 if cu_seqlens is not None else q.shape[0]
        shapes = [(n, q.shape[2], q.shape[3], v.shape[3])]
    inputs = [q, k, v, g, beta, w, initial_state] + ([cu_seqlens] if cu_seqlens is not None else [])
    r = _run("gated_deltanet2", inputs, 2, allocator, stream,
             state_shapes=shapes, prepare=prepare,
             scale=scale, use_qk_l2norm_in_kernel=int(bool(use_qk_l2norm_in_kernel)),
             output_final_state=int(bool(output_final_state)), use_gate_in_kernel=int(bool(use_gate_in_kernel)),
             has_cu_seqlens=int(cu_seqlens is not None), state_v_first=int(bool(state_v_first)))
    if prepare:
        if shapes is not None:
            r._result = (r.out, r.states[0])
        return r
    return (r[0], r[1][0]) if shapes is not None else r


def softmax_cpu(x, axis: int = -1):
    """SoftmaxCPU (CPU execution provider): softmax of a host fp32 array along
    ``axis`` (reference: softmax_cpu_ort.cpp:20-114).  Returns a new float32
    NumPy array of the input's shape."""
    import numpy as np
    a = np.asarray(x, dtype=np.float32, order="C")   # keeps rank 0 (ascontiguousarray would not)
    out = np.empty_like(a)
    shape = (ctypes.c_int64 * max(1, a.ndim))(*a.shape)
    err = ctypes.create_string_buffer(512)
    st = lib().xm_softmax_cpu(a.ctypes.data if a.size else None, shape, a.ndim, int(axis),
                              out.ctypes.data if out.size else None, err, len(err))
    _check(st, err)
    return out
