"""ctypes binding of libeth_amd.so (the C-ABI declared in include/eth_amd.h).

The product path has no fallback: if the library is missing or a call fails,
an exception is raised.  Tensors cross the boundary as raw device addresses;
the current torch stream is passed as the hipStream_t.
"""

import ctypes
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libeth_amd.so"

ETH_OK, ETH_ERR_INVALID, ETH_ERR_HIP = 0, 1, 2
ETH_F32, ETH_F16, ETH_BF16 = 0, 1, 2

CHUNK_ELEMS = 16384
CHUNK_NORM, CHUNK_SHADOWED = 1, 2
UNPACK_WRITEBACK, UNPACK_UNSCALE, UNPACK_STATS = 1, 2, 4
STATS_SCALED_OVERFLOW = 8

# struct eth_chunk (40 bytes)
CHUNK_DTYPE = np.dtype(
    {
        "names": ["src", "dst", "src_stride", "rows", "row_len", "scale", "flags"],
        "formats": ["<u8", "<i8", "<i8", "<i4", "<i4", "<f4", "<i4"],
        "offsets": [0, 8, 16, 24, 28, 32, 36],
        "itemsize": 40,
    }
)
# struct eth_bucket (40 bytes)
BUCKET_DTYPE = np.dtype(
    {
        "names": ["chunks", "n_chunks", "payload", "partial_base", "dtype", "reserved"],
        "formats": ["<u8", "<i8", "<u8", "<i8", "<i4", "<i4"],
        "offsets": [0, 8, 16, 24, 32, 36],
        "itemsize": 40,
    }
)
# struct eth_adam_tensor (64 bytes)
ADAM_TENSOR_DTYPE = np.dtype(
    {
        "names": ["param", "grad", "exp_avg", "exp_avg_sq", "model", "numel", "lr", "weight_decay"],
        "formats": ["<u8", "<u8", "<u8", "<u8", "<u8", "<i8", "<f8", "<f8"],
        "offsets": [0, 8, 16, 24, 32, 40, 48, 56],
        "itemsize": 64,
    }
)
# struct eth_adam_chunk (16 bytes)
ADAM_CHUNK_DTYPE = np.dtype(
    {"names": ["tensor", "n", "start"], "formats": ["<i4", "<i4", "<i8"], "offsets": [0, 4, 8], "itemsize": 16}
)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_F64 = ctypes.c_double

# name -> argtypes; every function returns int status except the two noted.
SIGNATURES = {
    "eth_fill_f32": [_P, _I64, _F32, _P],
    "eth_bucket_pack": [_P, _I64, _P, _I32, _P],
    "eth_bucket_unpack": [_P, _I64, _P, _I32, _F32, _F32, _I32, _P, _P, _I64, _P],
    "eth_bucket_sync_local": [_P, _I64, _F32, _F32, _I32, _P, _P, _P, _I64, _P],
    "eth_grad_stats": [_P, _I64, _F32, _I32, _P, _P, _I64, _P],
    "eth_tied_grad_sum_stats": [_P, _I64, _P, _P, _F32, _P, _P, _I64, _P],
    "eth_widen_grad_stats": [_P, _I64, _P, _I32, _F32, _I32, _P, _P, _I64, _P],
    "eth_grad_norm_finalize": [_P, _I64, _F64, _P, _P],
    "eth_adam_step": [_P, _P, _I64, _F64, _F64, _F64, _I64, _I32, _P, _P, _P],
    "eth_gemm": [_P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I64, _I64, _I32, _I32, _F32, _P],
    "eth_gemm_splitk": [_P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P, _P],
    "eth_ln_fwd": [_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _I32, _P],
    "eth_ln_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _P],
    "eth_ln_fwd_sb": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F32, _I32, _P],
    "eth_ln_bwd_sb": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _P],
    "eth_bias_gelu_fwd": [_P, _P, _P, _I64, _I64, _I32, _P],
    "eth_bias_gelu_bwd": [_P, _P, _P, _P, _I64, _I64, _I32, _P],
    "eth_bias_dropout_add_fwd": [_P, _P, _P, _P, _I64, _I64, _F32, ctypes.c_uint64, _I32, _P],
    "eth_bda_ln_fwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F32, ctypes.c_uint64, _F32, _I32, _P],
    "eth_dropout_bwd": [_P, _P, _I64, _I64, _F32, ctypes.c_uint64, _I32, _P],
    "eth_col_sum": [_P, _I64, _I64, _I64, _P, _P, _I32, _I32, _P],
    "eth_ln_bwd_residual": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _P],
    "eth_bias_gelu_bwd_dbias": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _P],
    "eth_reduce_partials": [_P, _I64, _I64, _I64, _P, _I32, _P],
}
SIGNATURES["eth_embedding_fwd"] = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P]
SIGNATURES["eth_embedding_bwd"] = [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P]
SIGNATURES["eth_embedding_bwd_noalloc"] = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P]
SIGNATURES["eth_xent_fwd"] = [_P, _I64, _P, _P, _P, _I64, _I64, _P, _I32, _P]
SIGNATURES["eth_xent_bwd"] = [_P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _P]
SIGNATURES["eth_tied_grad_sum"] = [_P, _P, _I64, _P]
SIGNATURES["eth_tied_grad_sum_half"] = [_P, _P, _I64, _I32, _P]
SIGNATURES["eth_synthetic_batch"] = [_P, _I64, _I64, _I64, _P, _P, _P, _P]
SIGNATURES["eth_attn_fwd"] = [_P, _P, _P, _P, _P, _P, _P]
SIGNATURES["eth_attn_bwd"] = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]


class AttnDesc(ctypes.Structure):
    """struct eth_attn_desc (include/eth_amd.h)."""

    _fields_ = [
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("seq", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("q_strides", ctypes.c_int64 * 3),
        ("k_strides", ctypes.c_int64 * 3),
        ("v_strides", ctypes.c_int64 * 3),
        ("o_strides", ctypes.c_int64 * 3),
        ("do_strides", ctypes.c_int64 * 3),
        ("dq_strides", ctypes.c_int64 * 3),
        ("dk_strides", ctypes.c_int64 * 3),
        ("dv_strides", ctypes.c_int64 * 3),
    ]


# functions returning a value instead of a status
VALUE_SIGNATURES = {
    "eth_ln_bwd_workspace": ([_I64, _I64], _I64),
    "eth_ln_bwd_groups": ([_I64, _I64], _I64),
    "eth_bias_gelu_bwd_workspace": ([_I64, _I64], _I64),
    "eth_col_sum_workspace": ([_I64, _I64], _I64),
    "eth_gemm_splitk_workspace": ([_I64, _I64, _I32], _I64),
    "eth_embedding_bwd_workspace": ([_I64, _I64], _I64),
}
GEMM_ACCUMULATE, GEMM_BIAS = 1, 2

_lib = None


class EthError(RuntimeError):
    pass


def load(path=None):
    """Load the shared library once; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(path or os.environ.get("ETH_AMD_LIB", LIB_PATH))
    if not path.exists():
        raise EthError(
            f"{path} is missing: build it with `python -m eth_amd.build` "
            "(the HIP path has no CPU fallback)"
        )
    lib = ctypes.CDLL(str(path))
    lib.eth_abi_version.restype = ctypes.c_int
    lib.eth_abi_version.argtypes = []
    lib.eth_last_error.restype = ctypes.c_char_p
    lib.eth_last_error.argtypes = []
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = argtypes
    for name, (argtypes, restype) in VALUE_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def exported_symbols():
    return ["eth_abi_version", "eth_last_error", *SIGNATURES, *VALUE_SIGNATURES]


def value(name, *args):
    return getattr(load(), name)(*args)


def call(name, *args):
    lib = load()
    status = getattr(lib, name)(*args)
    if status != ETH_OK:
        msg = lib.eth_last_error().decode(errors="replace")
        if status == ETH_ERR_INVALID:
            raise ValueError(f"{name}: {msg}")
        raise EthError(f"{name}: {msg}")


def dtype_code(torch_dtype):
    import torch

    codes = {torch.float32: ETH_F32, torch.float16: ETH_F16, torch.bfloat16: ETH_BF16}
    if torch_dtype not in codes:
        raise ValueError(f"unsupported dtype {torch_dtype}")
    return codes[torch_dtype]


def stream_ptr(device=None):
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr()) if tensor is not None else ctypes.c_void_p(0)


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("eth_amd kernels require tensors on the GPU (no CPU fallback)")


def table_to_device(array, device):
    """Copy a numpy structured table to device memory (uint8 tensor)."""
    import torch

    host = torch.from_numpy(np.ascontiguousarray(array).view(np.uint8).copy())
    return host.to(device=device, non_blocking=False)
