"""ctypes declarations of the C ABI in include/xmetai_recurrent.h."""

from __future__ import annotations

import ctypes
import os

XM_MAX_RANK = 8
XM_ELEM_FLOAT = 1
XM_ELEM_INT64 = 7   # cu_seqlens
XM_ELEM_FLOAT16 = 10
XM_ELEM_BFLOAT16 = 16

XM_OK = 0
XM_ERR_INVALID_ARGUMENT = 1
XM_ERR_UNSUPPORTED = 2
XM_ERR_DEVICE = 3
XM_ERR_ALLOC = 4

STATUS_NAMES = {
    XM_OK: "XM_OK",
    XM_ERR_INVALID_ARGUMENT: "XM_ERR_INVALID_ARGUMENT",
    XM_ERR_UNSUPPORTED: "XM_ERR_UNSUPPORTED",
    XM_ERR_DEVICE: "XM_ERR_DEVICE",
    XM_ERR_ALLOC: "XM_ERR_ALLOC",
}

LIB_NAME = "libxmetai_recurrent.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


class XmTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("shape", ctypes.c_int64 * XM_MAX_RANK),
        ("rank", ctypes.c_int32),
        ("elem_type", ctypes.c_int32),
    ]


ALLOC_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t)
FREE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p)


class XmAllocator(ctypes.Structure):
    _fields_ = [("ctx", ctypes.c_void_p), ("alloc", ALLOC_FN), ("free", FREE_FN)]


class SelectiveScanAttrs(ctypes.Structure):
    _fields_ = [("delta_softplus", ctypes.c_int64), ("return_last_state", ctypes.c_int64)]


class Mamba3SisoAttrs(ctypes.Structure):
    _fields_ = [
        ("chunk_size", ctypes.c_int64),
        ("has_d", ctypes.c_int64),
        ("has_z", ctypes.c_int64),
        ("return_final_states", ctypes.c_int64),
        ("has_input_states", ctypes.c_int64),
        ("has_cu_seqlens", ctypes.c_int64),
    ]


class GatedDeltaNet2Attrs(ctypes.Structure):
    _fields_ = [
        ("scale", ctypes.c_float),
        ("use_qk_l2norm_in_kernel", ctypes.c_int64),
        ("output_final_state", ctypes.c_int64),
        ("use_gate_in_kernel", ctypes.c_int64),
        ("has_cu_seqlens", ctypes.c_int64),
        ("state_v_first", ctypes.c_int64),
    ]


# (op prefix, attrs struct, number of inputs; Mamba3SisoFn takes 15 with has_input_states)
OPS = {
    "selective_scan": (SelectiveScanAttrs, 8),
    "mamba3_siso": (Mamba3SisoAttrs, 11),
    "gated_deltanet2": (GatedDeltaNet2Attrs, 7),
}

# Ops with a second entry point that also writes the recurrent state after the
# last token: op prefix -> (the attribute that asks for it, number of state buffers).
STATE_OUTPUTS = {"selective_scan": ("return_last_state", 1), "gated_deltanet2": ("output_final_state", 1),
                 "mamba3_siso": ("return_final_states", 4)}
MAMBA3_INPUTS_WITH_STATES = 15
MAMBA3_INPUTS_PACKED = 16        # cu_seqlens at input 15
GDN2_INPUTS_PACKED = 8           # cu_seqlens at input 7

# Every symbol include/xmetai_recurrent.h declares.
EXPORTED_SYMBOLS = [
    f"xm_{op}_{fn}" for op in OPS for fn in ("attrs_default", "check_attrs", "validate", "forward")
] + [f"xm_{op}_forward_states" for op in STATE_OUTPUTS] + ["xm_gated_deltanet2_forward_noalloc", "xm_softmax_cpu", "xm_set_kernel_override",
                                                              "xm_get_kernel_override", "xm_last_launches",
                                                              "xm_version"]

# Kernel-selection overrides (xm_set_kernel_override) and the values each accepts besides 0.
KERNEL_OVERRIDES = {"gdn2_path": (1,), "gdn2_pairwise": (1,), "gdn2_rows": (1, 2, 4), "m3_path": (1,),
                    "ss_lpc": (1, 2, 4, 8, 16), "ss_split": (1, 2), "gdn2_kpw4": (1,),
                    "gdn2_windowed": (1,), "gdn2_split": (1, 2), "gdn2_ct": (1, 2)}


def declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    T = ctypes.POINTER(XmTensor)
    for op, (attrs_t, _) in OPS.items():
        A = ctypes.POINTER(attrs_t)
        f = getattr(lib, f"xm_{op}_attrs_default")
        f.argtypes = [A]
        f.restype = None
        f = getattr(lib, f"xm_{op}_check_attrs")
        f.argtypes = [A, ctypes.c_char_p, ctypes.c_size_t]
        f.restype = ctypes.c_int
        f = getattr(lib, f"xm_{op}_validate")
        f.argtypes = [T, ctypes.c_size_t, A, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32),
                      ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p, ctypes.c_size_t]
        f.restype = ctypes.c_int
        f = getattr(lib, f"xm_{op}_forward")
        f.argtypes = [T, ctypes.c_size_t, A, ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(XmAllocator),
                      ctypes.c_char_p, ctypes.c_size_t]
        f.restype = ctypes.c_int
        if op in STATE_OUTPUTS:
            nstate = STATE_OUTPUTS[op][1]
            f = getattr(lib, f"xm_{op}_forward_states")
            f.argtypes = [T, ctypes.c_size_t, A, ctypes.c_void_p] + [ctypes.c_void_p] * nstate + [
                ctypes.c_void_p, ctypes.POINTER(XmAllocator), ctypes.c_char_p, ctypes.c_size_t]
            f.restype = ctypes.c_int
    f = lib.xm_gated_deltanet2_forward_noalloc
    f.argtypes = [T, ctypes.c_size_t, ctypes.POINTER(GatedDeltaNet2Attrs), ctypes.c_void_p, ctypes.c_void_p,
                  ctypes.c_char_p, ctypes.c_size_t]
    f.restype = ctypes.c_int
    lib.xm_softmax_cpu.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    lib.xm_softmax_cpu.restype = ctypes.c_int
    lib.xm_set_kernel_override.argtypes = [ctypes.c_char_p, ctypes.c_int64, ctypes.c_char_p, ctypes.c_size_t]
    lib.xm_set_kernel_override.restype = ctypes.c_int
    lib.xm_get_kernel_override.argtypes = [ctypes.c_char_p]
    lib.xm_get_kernel_override.restype = ctypes.c_int64
    lib.xm_last_launches.argtypes = []
    lib.xm_last_launches.restype = ctypes.c_char_p
    lib.xm_version.argtypes = []
    lib.xm_version.restype = ctypes.c_char_p
    return lib
