"""ctypes binding of libatlas_mem.so (the C ABI in include/atlas_mem.h).

The structs below mirror the header field by field. Loading fails loudly when the library
has not been built: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libatlas_mem.so")

ABI_VERSION = 1

OK = 0
ERR_UNSUPPORTED = 6
ERR_SCRATCH = 10

DT_F32 = 0
DT_BF16 = 1

GATE_NONE = 0
GATE_TOKEN = 1
GATE_LAG = 2

MAP_OFF = 0
MAP_ELEMENTWISE = 1

# every symbol include/atlas_mem.h declares
EXPORTED_SYMBOLS = (
    "atlas_mem_abi_version",
    "atlas_mem_strerror",
    "atlas_mem_validate",
    "atlas_mem_saved_bytes",
    "atlas_mem_bwd_workspace_bytes",
    "atlas_mem_fwd",
    "atlas_mem_bwd",
    "atlas_mem_bwd_noalloc",
    "atlas_mem_noalloc_scratch_bytes",
    "atlas_mem_step",
    "atlas_mem_step_factored",
    "atlas_buffer_factors",
    "atlas_buffer_expand",
    "atlas_scan_fwd",
    "atlas_scan_bwd",
    "atlas_window_sum",
    "atlas_affine_scan_fwd",
    "atlas_affine_scan_bwd",
    "atlas_affine_scan_workspace_bytes",
    "atlas_tensor_map_fwd",
    "atlas_tensor_map_bwd",
    "atlas_tensor_map_symmetrize",
    "atlas_tensor_map_fwd_sym",
    "atlas_tensor_map_bwd_sym",
    "atlas_block_split",
    "atlas_block_merge",
    "atlas_block_parts",
    "atlas_partials_sum",
    "atlas_replicas",
    "atlas_prologue_num_workgroups",
    "atlas_prologue_fwd",
    "atlas_prologue_bwd",
    "atlas_heads_fwd",
    "atlas_heads_bwd",
    "atlas_linear_batch",
    "atlas_linear_wgrad_workspace_bytes",
    "atlas_linear_wgrad",
    "atlas_linear_wgrad_batch_workspace_bytes",
    "atlas_linear_wgrad_batch",
    "atlas_mem_profile_enable",
    "atlas_mem_profile_read",
    "atlas_mem_kernel_name",
    "atlas_mem_mfma_selftest",
)

NKERNELS = 14


class Problem(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "abi_version", "bh", "seq_len", "d_k", "d_v", "window", "momentum", "gate_mode",
        "map_mode", "map_degree", "has_buffer", "clamp_every", "clamp_final", "dtype")]


class FwdArgs(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "k", "q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0", "buffer_in",
        "y", "S_T", "Z_T", "buffer_out")]


class BwdArgs(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "k", "q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0", "buffer_in",
        "dy", "dS_T", "dZ_T", "dbuffer_out",
        "dk", "dq", "dv", "dlr", "ddecay", "dbeta", "dgate",
        "dS_ref", "dS0", "dZ0", "dbuffer_in")]


_LIB = None


class LibraryMissing(RuntimeError):
    pass


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and type the C ABI. Raises LibraryMissing if the .so is not built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise LibraryMissing(
            f"{p} is not built; run `python -m atlas_rnn_amd.build` (hipcc, gfx950). "
            "atlas_rnn_amd has no CPU fallback.")
    lib = ctypes.CDLL(p)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    P = ctypes.POINTER(Problem)
    lib.atlas_mem_abi_version.restype = i32
    lib.atlas_mem_abi_version.argtypes = []
    lib.atlas_mem_strerror.restype = ctypes.c_char_p
    lib.atlas_mem_strerror.argtypes = [i32]
    lib.atlas_mem_validate.restype = i32
    lib.atlas_mem_validate.argtypes = [P]
    lib.atlas_mem_saved_bytes.restype = sz
    lib.atlas_mem_saved_bytes.argtypes = [P]
    lib.atlas_mem_bwd_workspace_bytes.restype = sz
    lib.atlas_mem_bwd_workspace_bytes.argtypes = [P]
    lib.atlas_mem_fwd.restype = i32
    lib.atlas_mem_fwd.argtypes = [P, ctypes.POINTER(FwdArgs), vp, vp]
    lib.atlas_mem_step.restype = i32
    lib.atlas_mem_step.argtypes = [P, ctypes.POINTER(FwdArgs), vp]
    lib.atlas_mem_step_factored.restype = i32
    lib.atlas_mem_step_factored.argtypes = [P, ctypes.POINTER(FwdArgs), vp, vp, vp]
    lib.atlas_buffer_factors.restype = i32
    lib.atlas_buffer_factors.argtypes = [P] + [vp] * 7
    lib.atlas_buffer_expand.restype = i32
    lib.atlas_buffer_expand.argtypes = [i32] * 4 + [vp] * 3
    lib.atlas_mem_bwd.restype = i32
    lib.atlas_mem_bwd.argtypes = [P, ctypes.POINTER(BwdArgs), vp, vp, sz, vp]
    lib.atlas_mem_bwd_noalloc.restype = i32
    lib.atlas_mem_bwd_noalloc.argtypes = [P, ctypes.POINTER(BwdArgs), vp, vp]
    lib.atlas_mem_noalloc_scratch_bytes.restype = sz
    lib.atlas_mem_noalloc_scratch_bytes.argtypes = []
    lib.atlas_scan_fwd.restype = i32
    lib.atlas_scan_fwd.argtypes = [i32, i64, i64, i64, vp, vp, vp, vp, vp]
    lib.atlas_scan_bwd.restype = i32
    lib.atlas_scan_bwd.argtypes = [i32, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.atlas_window_sum.restype = i32
    lib.atlas_window_sum.argtypes = [i32, i64, i64, i64, i32, i32, vp, vp, vp]
    lib.atlas_affine_scan_fwd.restype = i32
    lib.atlas_affine_scan_fwd.argtypes = [i32, i32, i32, i32, vp, vp, vp, vp, vp, sz, vp]
    lib.atlas_affine_scan_bwd.restype = i32
    lib.atlas_affine_scan_bwd.argtypes = [i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.atlas_affine_scan_workspace_bytes.restype = sz
    lib.atlas_affine_scan_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.atlas_tensor_map_fwd.restype = i32
    lib.atlas_tensor_map_fwd.argtypes = [i32, i64, i32, i32, i32, vp, vp, vp, vp, vp]
    lib.atlas_tensor_map_bwd.restype = i32
    lib.atlas_tensor_map_bwd.argtypes = [i32, i64, i32, i32, i32, vp, vp, vp, vp, vp, vp]
    lib.atlas_tensor_map_symmetrize.restype = i32
    lib.atlas_tensor_map_symmetrize.argtypes = [i32, i32, i32, vp, vp, vp, vp]
    lib.atlas_tensor_map_fwd_sym.restype = i32
    lib.atlas_tensor_map_fwd_sym.argtypes = [i32, i64, i32, i32, i32, vp, vp, vp, vp, vp]
    lib.atlas_tensor_map_bwd_sym.restype = i32
    lib.atlas_tensor_map_bwd_sym.argtypes = [i32, i64, i32, i32, i32, vp, vp, vp, vp, vp, vp]
    lib.atlas_block_split.restype = i32
    lib.atlas_block_split.argtypes = [i32] * 5 + [vp] * 8
    lib.atlas_block_merge.restype = i32
    lib.atlas_block_merge.argtypes = [i32] * 5 + [vp] * 10
    lib.atlas_block_parts.restype = i32
    lib.atlas_block_parts.argtypes = [i32]
    f32 = ctypes.c_float
    lib.atlas_partials_sum.restype = i32
    lib.atlas_partials_sum.argtypes = [i32, i32, ctypes.POINTER(i32), ctypes.POINTER(vp), ctypes.POINTER(vp),
                                       ctypes.POINTER(i32), vp]
    lib.atlas_replicas.restype = i32
    lib.atlas_replicas.argtypes = [i32, i32, i32, i32, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(vp),
                                   ctypes.POINTER(vp), vp]
    lib.atlas_prologue_num_workgroups.restype = i32
    lib.atlas_prologue_num_workgroups.argtypes = [i32, i32]
    lib.atlas_prologue_fwd.restype = i32
    lib.atlas_prologue_fwd.argtypes = [i32, i32, i32, i32, i32, f32] + [vp] * 11
    lib.atlas_prologue_bwd.restype = i32
    lib.atlas_prologue_bwd.argtypes = [i32, i32, i32, i32, i32] + [vp] * 14
    lib.atlas_heads_fwd.restype = i32
    lib.atlas_heads_fwd.argtypes = [i32] * 6 + [vp] * 12
    lib.atlas_heads_bwd.restype = i32
    lib.atlas_heads_bwd.argtypes = [i32] * 6 + [vp] * 17
    lib.atlas_linear_batch.restype = i32
    lib.atlas_linear_batch.argtypes = [i32, i32, i64, ctypes.POINTER(i32), ctypes.POINTER(i32),
                                       ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.POINTER(vp), vp]
    lib.atlas_linear_wgrad_workspace_bytes.restype = i64
    lib.atlas_linear_wgrad_workspace_bytes.argtypes = [i64, i32, i32]
    lib.atlas_linear_wgrad.restype = i32
    lib.atlas_linear_wgrad.argtypes = [i32, i64, i32, i32, vp, vp, vp, vp, i64, vp]
    lib.atlas_linear_wgrad_batch_workspace_bytes.restype = i64
    lib.atlas_linear_wgrad_batch_workspace_bytes.argtypes = [i32, i64, ctypes.POINTER(i32), ctypes.POINTER(i32)]
    lib.atlas_linear_wgrad_batch.restype = i32
    lib.atlas_linear_wgrad_batch.argtypes = [i32, i32, i64, ctypes.POINTER(i32), ctypes.POINTER(i32),
                                             ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.POINTER(vp), vp, i64, vp]
    lib.atlas_mem_profile_enable.restype = i32
    lib.atlas_mem_profile_enable.argtypes = [i32]
    lib.atlas_mem_profile_read.restype = i32
    lib.atlas_mem_profile_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_longlong), i32, i32]
    lib.atlas_mem_kernel_name.restype = ctypes.c_char_p
    lib.atlas_mem_kernel_name.argtypes = [i32]
    lib.atlas_mem_mfma_selftest.restype = i32
    lib.atlas_mem_mfma_selftest.argtypes = [i32, vp, vp, vp, vp]
    if lib.atlas_mem_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {lib.atlas_mem_abi_version()} != {ABI_VERSION}")
    if path is None:
        _LIB = lib
    return lib


def check(status: int, what: str) -> None:
    if status != OK:
        msg = load().atlas_mem_strerror(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")
