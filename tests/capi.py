"""ctypes views of the kernel library's C ABI (include/mgc_hip.h) for tests that call its entry
points directly, and the few HIP runtime calls they need for their own device buffers."""

from __future__ import annotations

import ctypes

import numpy as np

MGC_OK, MGC_ERR_GATHER_INDEX, MGC_ERR_HIP, MGC_ERR_ARGS = 0, 1, 2, 3
MGC_OP_STRIDED, MGC_OP_CONV_NHWC, MGC_OP_CONV_NCHW = 0, 1, 2
ACTS = ("none", "relu", "clip", "gelu", "gelu_tanh", "tanh", "sigmoid")  # MGC_ACT_* order
GEMM_FAMILIES = {"auto": 0, "tiled": 1, "quarter": 2, "narrow": 3, "wsplit": 4, "wsplit16": 5, "stream": 6,
                 "register": 7}  # MGC_GEMM_*


class Operand(ctypes.Structure):
    """mgc_hip_operand."""

    _fields_ = [("kind", ctypes.c_int), ("p", ctypes.c_void_p), ("rs", ctypes.c_long), ("cs", ctypes.c_long)] + [
        (n, ctypes.c_int) for n in ("H", "W", "C", "KH", "KW", "SH", "SW", "DH", "DW", "PT", "PL", "OH", "OW", "cg")
    ]


class GemmArgs(ctypes.Structure):
    """mgc_hip_gemm_args."""

    _fields_ = [
        ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
        ("a", Operand), ("b", Operand),
        ("c", ctypes.c_void_p), ("ldc", ctypes.c_long),
        ("alpha", ctypes.c_float), ("beta", ctypes.c_float),
        ("bias", ctypes.c_void_p), ("bias_mode", ctypes.c_int),
        ("res", ctypes.c_void_p), ("ldr", ctypes.c_long),
        ("act", ctypes.c_int), ("lo", ctypes.c_float), ("hi", ctypes.c_float),
        ("batch_rank", ctypes.c_int), ("batch_dims", ctypes.c_int * 4),
        ("a_bs", ctypes.c_long * 4), ("b_bs", ctypes.c_long * 4), ("c_bs", ctypes.c_long * 4), ("r_bs", ctypes.c_long * 4),
        ("workspace", ctypes.c_void_p), ("workspace_floats", ctypes.c_long),
        ("split_k", ctypes.c_int),
        ("a2", Operand), ("k1", ctypes.c_int),
        ("kernel", ctypes.c_int),
    ]


class Hip:
    """hipMalloc'd buffers owned by a test, freed together."""

    def __init__(self) -> None:
        self.lib = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)  # the runtime libmgc_hip.so links
        self.lib.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.lib.hipFree.argtypes = [ctypes.c_void_p]
        self.lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.buffers: list[ctypes.c_void_p] = []

    def check(self, code: int, what: str) -> None:
        assert code == 0, f"{what} failed with {code}"

    def alloc(self, nbytes: int) -> int:
        ptr = ctypes.c_void_p()
        self.check(self.lib.hipMalloc(ctypes.byref(ptr), max(nbytes, 4)), "hipMalloc")
        self.buffers.append(ptr)
        return ptr.value

    def put(self, ptr: int, array: np.ndarray) -> int:
        array = np.ascontiguousarray(array)
        self.check(self.lib.hipMemcpy(ctypes.c_void_p(ptr), array.ctypes.data, array.nbytes, 1), "hipMemcpy H2D")
        return ptr

    def upload(self, array: np.ndarray) -> int:
        array = np.ascontiguousarray(array)
        return self.put(self.alloc(array.nbytes), array)

    def empty(self, nbytes: int) -> int:
        return self.upload(np.full(nbytes // 4, np.nan, np.float32))

    def download(self, ptr: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.check(self.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")
        self.check(self.lib.hipMemcpy(out.ctypes.data, ctypes.c_void_p(ptr), out.nbytes, 2), "hipMemcpy D2H")
        return out

    def free(self) -> None:
        for ptr in self.buffers:
            self.lib.hipFree(ptr)
        self.buffers.clear()


def bind(lib) -> None:
    """Argument and result types of the entry points the tests call."""
    lib.mgc_hip_last_error.restype = ctypes.c_char_p
    lib.mgc_hip_exec_create.restype = ctypes.c_void_p
    lib.mgc_hip_exec_create.argtypes = [ctypes.c_void_p]
    lib.mgc_hip_exec_status.restype = ctypes.c_int
    lib.mgc_hip_exec_status.argtypes = [ctypes.c_void_p]
    lib.mgc_hip_exec_destroy.argtypes = [ctypes.c_void_p]
    lib.mgc_hip_gemm.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.mgc_hip_gemm_noalloc.restype = ctypes.c_int
    lib.mgc_hip_gemm_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.mgc_hip_gemm_workspace.restype = ctypes.c_long
    lib.mgc_hip_gemm_workspace.argtypes = [ctypes.c_int] * 4
