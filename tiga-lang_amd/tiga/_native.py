"""ctypes binding of libtgx_hip.so (the C ABI declared in include/tgx.h).

Every call passes raw device pointers from Torch tensors and Torch's current
HIP stream; a non-zero status raises ``RuntimeError`` with the library's
message, as the reference runtime binding does
(python/tiga/runtime/__init__.py:279-285).  The library is loaded from the
package's own ``_lib`` directory only; nothing here falls back to another
implementation when it is missing.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtgx_hip.so"
_lib = None

c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p
P = ctypes.POINTER


class RowPlan(ctypes.Structure):
    """Mirror of ``tgx_row_plan``."""

    _fields_ = [
        ("n_rows", c_i64),
        ("n_empty", c_i64),
        ("n_wave", c_i64),
        ("n_split", c_i64),
        ("n_chunks", c_i64),
        ("wave_max", ctypes.c_int32),
        ("chunk_edges", ctypes.c_int32),
        ("rows_dev", c_vp),
        ("chunk_offsets_dev", c_vp),
    ]


class EdgeMlp(ctypes.Structure):
    """Mirror of ``tgx_edge_mlp``."""

    _fields_ = [("n_layers", ctypes.c_int32), ("width", ctypes.c_int32),
                ("act", ctypes.c_int32 * 3), ("act_param", ctypes.c_float * 3),
                ("weights_dev", c_vp), ("n_segments", ctypes.c_int32),
                ("seg_role", ctypes.c_int32 * 4), ("seg_width", ctypes.c_int32 * 4),
                ("seg_stride", ctypes.c_int64 * 4), ("seg_dev", c_vp * 4),
                ("out_width", ctypes.c_int32 * 3), ("act_param2", ctypes.c_float * 3),
                ("norm", ctypes.c_int32 * 3), ("norm_eps", ctypes.c_float * 3)]


# tgx_abi_version() of the library these signatures and structs mirror.
ABI_VERSION = 13


# name -> argtypes (all return int status except where noted)
_SIGNATURES: dict[str, list] = {
    "tgx_abi_version": [],
    "tgx_destination_index": [c_vp, c_int, c_i64, c_i64, c_vp, c_int, c_vp],
    "tgx_csr_transpose_workspace": [c_i64, c_i64, c_i64, P(c_size)],
    "tgx_csr_transpose": [c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
                          c_vp, c_vp, c_size, c_vp],
    "tgx_coo_to_csr_workspace": [c_i64, c_i64, c_i64, P(c_size)],
    "tgx_coo_to_csr": [c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
                       c_vp, c_size, c_vp],
    "tgx_varlen_csr_workspace": [c_i64, P(c_size)],
    "tgx_varlen_csr": [c_vp, c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_vp, c_vp, c_size,
                       c_vp],
    "tgx_plan_degree_bins_workspace": [c_i64, c_int, P(c_size)],
    "tgx_plan_degree_bins": [c_vp, c_int, c_i64, P(c_i64), c_int, c_vp, P(c_i64), c_vp,
                             c_size, c_vp],
    "tgx_plan_split_chunks": [c_vp, c_int, c_vp, c_i64, ctypes.c_int32, c_vp, P(c_i64),
                              c_vp],
    "tgx_plan_reference_buckets": [c_i64, c_i64, c_i64, P(c_i64), c_int, P(c_int),
                                   P(c_i64), P(c_i64), P(c_int), P(c_i64), P(c_int),
                                   P(c_i64), P(c_i64)],
    "tgx_partial_bytes": [P(RowPlan), c_i64, P(c_size)],
    "tgx_csr_sum_fwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_i64, c_i64,
                        c_i64, c_int, c_vp, c_vp],
    "tgx_csr_sum_bwd": [c_vp, c_vp, c_vp, P(RowPlan), c_vp, c_vp, c_vp, c_vp, c_vp,
                        c_i64, c_i64, c_i64, c_int, c_vp, c_vp],
    "tgx_csr_edge_dot": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                         c_int, c_vp],
    "tgx_gat_fwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, c_f32, c_vp,
                    c_vp, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_vp, c_vp],
    "tgx_gat_bwd_workspace": [P(RowPlan), P(RowPlan), c_i64, c_int, c_int, c_int, c_int,
                              P(c_size)],
    "tgx_gat_bwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, P(RowPlan), c_vp,
                    c_vp, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                    c_i64, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_size, c_vp],
    "tgx_dot_attn_fwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, c_f32, c_vp,
                         c_vp, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_vp],
    "tgx_dot_attn_fwd_noalloc": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp,
                                 c_f32, c_vp, c_vp, c_i64, c_i64, c_int, c_int, c_int, c_vp],
    "tgx_dot_attn_bwd_workspace": [P(RowPlan), P(RowPlan), c_i64, c_int, c_int, c_int,
                                   P(c_size)],
    "tgx_dot_attn_bwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, P(RowPlan),
                         c_i64, c_vp, c_vp, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp, c_vp,
                         c_vp, c_vp, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_size, c_vp],
    "tgx_attn_tasks": [c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp, P(c_i64)],
    "tgx_attn_fwd": [c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_vp, c_vp, c_vp, P(c_i64),
                     c_f32, c_f32, c_vp, c_vp, c_i64, c_i64, c_int, c_int, c_vp],
    "tgx_attn_bwd": [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_vp, c_vp,
                     P(c_i64), c_vp, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
                     c_int, c_int, c_vp],
    "tgx_attn_ds_tiles": [c_vp, c_vp, c_int, c_int, c_int, P(c_i64)],
    "tgx_attn_fwd_split_tasks": [c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp, P(c_i64), c_vp,
                                 P(c_i64), P(ctypes.c_int32), P(ctypes.c_int32)],
    "tgx_attn_fwd_split": [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, ctypes.c_int32, ctypes.c_int32,
                           c_int, c_int, c_vp, c_vp, c_vp, P(c_i64), c_f32, c_vp, c_vp, c_vp,
                           c_i64, c_i64, c_int, c_int, c_vp],
    "tgx_attn_bwd_stored": [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_vp, c_vp,
                            c_vp, P(c_i64), c_vp, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp,
                            c_vp, c_i64, c_i64, c_int, c_int, c_vp],
    "tgx_edge_mlp_scores": [c_vp, c_vp, c_int, c_i64, P(EdgeMlp), c_vp, c_vp],
    "tgx_edge_mlp_backward_workspace": [c_i64, P(EdgeMlp), P(c_size)],
    "tgx_edge_mlp_backward": [c_vp, c_vp, c_int, c_i64, P(EdgeMlp), c_vp, c_vp, P(c_vp),
                              c_vp, c_size, c_vp],
    "tgx_edge_mlp_attention_backward": [c_vp, c_vp, c_int, c_i64, P(EdgeMlp), c_vp, c_vp, c_vp,
                                        c_vp, ctypes.c_int32, c_vp, c_int, c_vp, P(c_vp), c_vp,
                                        c_size, c_vp],
    "tgx_edge_mlp_hidden": [c_vp, c_vp, c_int, c_i64, P(EdgeMlp), c_vp, ctypes.c_int32, c_vp],
    "tgx_edge_mlp_backward_seeded": [c_vp, c_vp, c_int, c_i64, P(EdgeMlp), c_vp,
                                     ctypes.c_int32, c_vp, P(c_vp), c_vp, c_size, c_vp],
    "tgx_segment_softmax_fwd": [c_vp, c_int, c_i64, c_vp, c_vp, c_vp, c_vp],
    "tgx_segment_softmax_bwd": [c_vp, c_int, c_i64, c_vp, c_vp, c_vp, c_vp],
    "tgx_segment_softmax_gather_fwd": [c_vp, c_vp, c_int, c_i64, c_vp, c_int, c_f32, c_vp,
                                       c_vp, c_vp],
    "tgx_segment_softmax_sum_fwd": [c_vp, c_vp, c_int, c_i64, c_vp, c_int, c_f32, c_vp, c_int,
                                    c_vp, c_vp, c_vp, c_vp],
    # CPU twins (include/tgx_cpu.h): host pointers, no stream.
    "tgx_cpu_set_threads": [c_int],
    "tgx_cpu_destination_index": [c_vp, c_int, c_i64, c_i64, c_vp, c_int],
    "tgx_cpu_csr_transpose": [c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp],
    "tgx_cpu_plan_degree_bins": [c_vp, c_int, c_i64, P(c_i64), c_int, c_vp, P(c_i64)],
    "tgx_cpu_plan_split_chunks": [c_vp, c_int, c_vp, c_i64, ctypes.c_int32, c_vp, P(c_i64)],
    "tgx_cpu_csr_sum_fwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_i64, c_i64,
                            c_i64, c_int],
    "tgx_cpu_csr_sum_bwd": [c_vp, c_vp, c_vp, P(RowPlan), c_vp, c_vp, c_vp, c_vp, c_vp, c_i64,
                            c_i64, c_i64, c_int],
    "tgx_cpu_csr_edge_dot": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_i64, c_i64,
                             c_i64, c_int],
    "tgx_cpu_gat_fwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, c_f32, c_vp,
                        c_vp, c_i64, c_i64, c_int, c_int, c_int],
    "tgx_cpu_gat_bwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, P(RowPlan),
                        c_vp, c_vp, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                        c_i64, c_i64, c_i64, c_int, c_int, c_int],
    "tgx_cpu_dot_attn_fwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, c_vp, c_f32,
                             c_vp, c_vp, c_i64, c_i64, c_int, c_int, c_int],
    "tgx_cpu_dot_attn_bwd": [c_vp, c_vp, c_int, P(RowPlan), c_vp, c_vp, c_vp, P(RowPlan),
                             c_vp, c_vp, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                             c_vp, c_i64, c_i64, c_int, c_int, c_int],
    "tgx_cpu_attn_fwd": [c_vp, c_vp, c_int, c_int, c_int, c_vp, c_vp, c_vp, P(c_i64), c_f32,
                         c_f32, c_vp, c_vp, c_i64, c_i64, c_int, c_int],
    "tgx_cpu_attn_bwd": [c_vp, c_vp, c_int, c_int, c_int, c_vp, c_vp, c_vp, P(c_i64), c_vp,
                         c_vp, c_vp, c_f32, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_int, c_int],
    "tgx_profile_begin": [],
    "tgx_profile_end": [],
    "tgx_profile_count": [],
    "tgx_profile_entry": [c_int, ctypes.c_char_p, c_int, P(c_i64), P(ctypes.c_double)],
}

_OPTIONAL: dict[str, list] = {}


def library_path() -> Path:
    return Path(os.environ.get("TGX_LIBRARY", _LIB_PATH))


def available() -> bool:
    return library_path().exists()


def lib():
    """Load (once) and return the native library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"libtgx_hip.so not found at {path}; build it with "
            "`python tiga-lang_amd/build_native.py` (or __graft_entry__.build())")
    handle = ctypes.CDLL(str(path))
    handle.tgx_status_string.restype = ctypes.c_char_p
    handle.tgx_status_string.argtypes = [c_int]
    handle.tgx_last_error.restype = ctypes.c_char_p
    handle.tgx_last_error.argtypes = []
    for name, argtypes in {**_SIGNATURES, **_OPTIONAL}.items():
        fn = getattr(handle, name, None)
        if fn is None:
            if name in _OPTIONAL:
                continue
            raise RuntimeError(f"{path} does not export {name}")
        fn.restype = c_int
        fn.argtypes = argtypes
    if handle.tgx_abi_version() != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI version {handle.tgx_abi_version()}, this package expects "
            f"{ABI_VERSION}; rebuild it with `python tiga-lang_amd/build_native.py`")
    _lib = handle
    return _lib


def call(name: str, *args) -> None:
    handle = lib()
    status = getattr(handle, name)(*args)
    if status != 0:
        raise_status(name, status)


def raise_status(name: str, status: int) -> None:
    """Raise the error a nonzero status of entry point `name` stands for."""
    handle = lib()
    message = handle.tgx_last_error().decode(errors="replace")
    kind = handle.tgx_status_string(status).decode()
    error = NotImplementedError if status == 2 else RuntimeError
    raise error(f"{name}: {kind}: {message}")


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES) + ["tgx_last_error", "tgx_status_string"]


def ptr(tensor) -> int | None:
    """Device pointer of a tensor (None for a missing optional operand)."""
    if tensor is None:
        return None
    return tensor.data_ptr()


def stream_of(tensor) -> int:
    """Torch's current stream on the tensor's device (a raw hipStream_t)."""
    import torch

    index = tensor.device.index
    if index is None:
        index = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2


def dtype_code(tensor) -> int:
    """TGX_DTYPE_* code of a bf16, fp16 or fp32 tensor."""
    import torch

    return {torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16,
            torch.float32: DTYPE_F32}[tensor.dtype]


def idx_bits(tensor) -> int:
    import torch

    return 64 if tensor.dtype == torch.int64 else 32


class KernelTimer:
    """Context manager over tgx_profile_begin/end: per-kernel launch counts
    and total milliseconds of every kernel the library launched inside it."""

    def __enter__(self):
        call("tgx_profile_begin")
        self.totals = {}
        return self

    def __exit__(self, *exc):
        call("tgx_profile_end")
        handle = lib()
        buf = ctypes.create_string_buffer(128)
        n_launch = c_i64()
        ms = ctypes.c_double()
        for i in range(handle.tgx_profile_count()):
            call("tgx_profile_entry", i, buf, 128, ctypes.byref(n_launch), ctypes.byref(ms))
            self.totals[buf.value.decode()] = (n_launch.value, ms.value)
        return False
