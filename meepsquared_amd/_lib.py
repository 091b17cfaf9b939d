"""The C ABI of libmlora.so (include/mlora.h), loaded with ctypes.

Every entry point returns an int status; `call` raises on a non-zero status with the library's own
message.  Tensors cross the boundary as raw device pointers (`ptr`), element counts and element
strides; the HIP stream is torch's current stream on the tensors' device.  There is no other
implementation behind these calls: without the library, importing this module fails.
"""

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "_lib" / "libmlora.so"

DT_BF16, DT_F32, DT_F16, DT_FP8_E4M3, DT_NF4, DT_NF4_KT = 0, 1, 2, 3, 4, 5
SCALE_NONE, SCALE_EXPERT, SCALE_ROW = 0, 1, 2

P = c_void_p
I64 = c_int64
# (name, argument types) for every entry point of include/mlora.h, in its order
SIGNATURES = {
    "mlora_version": (c_char_p, []),
    "mlora_last_error": (c_char_p, []),
    "mlora_route_topk": (c_int, [P, c_int, I64, I64, c_int, c_int, c_int, P, P, c_int, P]),
    "mlora_route_sort_workspace_bytes": (c_size_t, [I64, c_int]),
    "mlora_route_sort": (c_int, [P, I64, c_int, P, P, P, c_int, P, P, P, I64, P, c_size_t, P]),
    "mlora_route_sort_noalloc": (c_int, [P, I64, c_int, P, P, P, c_int, P, P, P, I64, P]),
    "mlora_tile_map": (c_int, [P, c_int, I64, c_int, P, P, P, I64, P]),
    "mlora_grouped_gemm": (c_int, [P, I64, I64, c_int, c_int,
                                   P, c_int, I64, I64, I64,
                                   P, c_int, I64, c_int,
                                   P, P, P, P, P,
                                   P, I64, I64,
                                   P, I64, I64, c_int, c_float,
                                   P, I64,
                                   P, I64, P, I64,
                                   P, c_int, P]),
    "mlora_grouped_gemm_gather": (c_int, [P, I64, I64, P, c_int, P, c_int, I64, c_int, c_int, P, c_int, I64, I64, I64,
                                          P, c_int, I64, P, I64, I64, P, I64, I64, c_int, c_float, P, I64,
                                          P, I64, P, I64, P, c_int, P]),
    "mlora_grouped_gemm_gather_q": (c_int, [P, I64, I64, P, c_int, P, c_int, I64, c_int, c_int,
                                            P, c_int, I64, I64, I64, P, c_int, I64, c_int,
                                            P, P, P, P, P,
                                            P, I64, I64, P, I64, I64, c_int, c_float, P, I64,
                                            P, I64, P, I64, P, c_int, P]),
    "mlora_grouped_gemm_gather_swiglu": (c_int, [P, I64, I64, P, c_int, I64, c_int, c_int,
                                                 P, c_int, I64, I64, I64, P, c_int, I64,
                                                 P, P, P, P, P,
                                                 P, I64, I64, P, I64, I64, c_int, c_float, P, I64,
                                                 P, I64, P, I64, P, I64, P, c_int, P]),
    "mlora_grouped_gemm_db_workspace_bytes": (c_size_t, [I64, c_int, c_int]),
    "mlora_grouped_gemm_db": (c_int, [P, I64, I64, P, c_int, P, c_int, I64, c_int, c_int,
                                      P, I64, I64, I64, P, c_int, I64,
                                      P, I64, I64, P, I64, I64, c_int, c_float, P, I64,
                                      P, I64, P, I64,
                                      P, I64, P, I64, I64, I64, P, c_size_t,
                                      P, c_int, P]),
    "mlora_grouped_reduce_workspace_bytes": (c_size_t, [I64, c_int, c_int, c_int]),
    "mlora_grouped_reduce": (c_int, [P, I64, P, I64, I64, c_int, c_int, c_float, P, c_int, P, I64, I64, I64, P, c_size_t,
                                     P]),
    "mlora_grouped_reduce_gather": (c_int, [P, I64, P, c_int, P, c_int, P, P, I64, I64, c_int, c_int, c_float, P,
                                            c_int, P, I64, I64, I64, P, c_size_t, P]),
    "mlora_gather_rows": (c_int, [P, I64, I64, P, I64, c_int, P, c_int, P, P]),
    "mlora_gather_rows_backward": (c_int, [P, I64, P, I64, c_int, P, c_int, P, P]),
    "mlora_swiglu": (c_int, [P, I64, I64, P, P]),
    "mlora_swiglu_backward": (c_int, [P, P, I64, I64, P, P]),
    "mlora_swiglu_backward_weighted": (c_int, [P, P, I64, I64, P, c_int, P, P, c_int, P, P, P]),
    "mlora_swiglu_backward_reduce_workspace_bytes": (c_size_t, [I64, I64, c_int]),
    "mlora_swiglu_backward_reduce": (c_int, [P, P, I64, I64, P, c_int, P, P, c_int, P, I64, c_float, P, I64, I64, I64,
                                             P, I64, c_float, P, I64, I64, I64, P, P, P, c_size_t, P]),
    "mlora_combine": (c_int, [P, I64, P, c_int, P, I64, c_int, P, c_int, P, P]),
    "mlora_combine_backward": (c_int, [P, P, I64, P, c_int, P, I64, c_int, P, c_int, P, P, P]),
    "mlora_scale_rows": (c_int, [P, I64, I64, I64, P, c_int, P, P, I64, P]),
    "mlora_swap_adapters": (c_int, [P, I64, I64, P, I64, I64, I64, I64, I64, I64, P, P, P]),
    "mlora_swap_adapters_two": (c_int, [P, I64, I64, P, I64, I64, I64, I64, I64, I64, P, P,
                                        P, I64, I64, P, I64, I64, I64, I64, I64, I64, P, P, P]),
    "mlora_transpose": (c_int, [P, I64, I64, I64, I64, I64, I64, P, P]),
    "mlora_transpose_u8": (c_int, [P, I64, I64, I64, I64, I64, I64, P, P]),
    "mlora_fp8_prep": (c_int, [P, I64, I64, c_int, c_int, P, I64, P, I64, P, I64, P, I64, I64, c_int, P, I64, P, c_int,
                               P]),
    "mlora_fp8_gemm": (c_int, [P, I64, P, I64, I64, c_int, c_int, c_int, P, I64, I64, P, c_int, I64, P, I64, P, I64, I64,
                               c_int, c_float, P, I64, P, I64, P, c_int, P]),
    "mlora_fp8_quantize": (c_int, [P, c_int, I64, I64, I64, c_int, c_int, P, P, P]),
    "mlora_fp8_dequantize": (c_int, [P, P, I64, I64, I64, c_int, c_int, P, c_int, P]),
    "mlora_nf4_workspace_bytes": (c_size_t, [I64]),
    "mlora_nf4_quantize": (c_int, [P, c_int, I64, P, P, P, P, P, P, P, c_size_t, P]),
    "mlora_nf4_dequantize": (c_int, [P, P, P, P, P, P, I64, P, c_int, P]),
    "mlora_nf4_transpose": (c_int, [P, P, P, P, P, I64, I64, I64, P, P, P]),
}


def _load():
    if not LIBRARY.exists():
        raise ImportError(f"{LIBRARY} is missing: build it with `python meepsquared_amd/_build.py` "
                          "(or __graft_entry__.build()); the operator has no other implementation")
    lib = ctypes.CDLL(str(LIBRARY))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class KernelError(RuntimeError):
    """A refusal or launch failure reported by libmlora."""


def call(name: str, *args) -> None:
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise KernelError(f"{name}: {lib.mlora_last_error().decode()}")


def ptr(t):
    """A tensor's device address (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream(device=None):
    """torch's current HIP stream on `device`, as the raw handle the library takes."""
    return torch.cuda.current_stream(device).cuda_stream


DTYPES = {torch.bfloat16: DT_BF16, torch.float32: DT_F32, torch.float16: DT_F16, torch.float8_e4m3fn: DT_FP8_E4M3}


def dtype_code(dtype) -> int:
    try:
        return DTYPES[dtype]
    except KeyError:
        raise TypeError(f"dtype {dtype} is not one the kernels take") from None


def require_gpu(*tensors):
    """Every tensor on a GPU, or a TypeError naming the first that is not (no CPU path exists)."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise TypeError(f"the kernels run on the GPU; got a tensor on {t.device}")
